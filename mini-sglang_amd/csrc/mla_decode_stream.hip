// Streaming absorbed-MLA decode for 64 query heads and pages of >= 32 tokens
// (the Kimi-K2 / DeepSeek-V3 decode shape on one GPU).
//
// Same plan, workspace and outputs as mla_decode_kernel, different schedule:
//  * The CTA's whole (request, token) range is ONE stream of 32-row tiles:
//    per piece, two tiles of queries (heads 0..31, 32..63: a query row has the
//    latent row's 576 dims, so it is staged like a KV row) and then the
//    piece's 32-token KV tiles. The 4-stage LDS ring keeps prefetching across
//    piece boundaries, queries included, so a new piece never drains it. The
//    page id of every KV tile and the bounds of every request of the range
//    are staged in LDS once, at CTA start.
//  * 4 waves = 2 head groups (32 heads each) x 2 halves for the scores, and
//    4 quarters of the value dims for the output. Wave w = (hg, th):
//      S^T[16 tokens (half th) x 32 heads] = K . Q^T     36 MFMAs, 18 K reads
//      softmax numerators of those 16 tokens, published as bf16 through LDS
//      so that every wave holds P for all 64 heads and 32 tokens
//      O^T[128 dims (quarter w) x 64 heads] += V^T . P^T 32 MFMAs, 16 V reads
//    Every staged K row is read by 2 waves and every V row by 1 wave, and no
//    MFMA or exponential is computed twice. The pair (hg, 0) / (hg, 1) agrees
//    on the exponent reference at the first tile of each piece; at its end the
//    row sums and references of all heads are exchanged, since every wave
//    normalises and writes its dims of all 64 heads.
//  * Barriers wait on LDS only, so the vector-memory operations in flight are
//    the ring's DMA loads and the output stores, both counted explicitly.
#include "mla_common.h"
#include "mla_device.h"

namespace mla {
namespace {

constexpr int kSWaves = 4;
constexpr int kSDma = kTileDma / kSWaves;  // DMA loads per wave per tile (9)
constexpr int kSKPrefetch = 6;             // K operands in flight
constexpr int kSVPrefetch = 4;             // V operand pairs in flight
constexpr float kSOverflowLog2 = 64.0f;    // see mla_decode.hip

// Position in the CTA's stream: request rb + r, piece [t0, t1); q < 2: the piece's query tile q
// (heads 32q .. +32), q == 2: the KV tile starting at token t.
struct Cursor {
  int r, t, t0, t1, q;
};

__global__ __launch_bounds__(256, 1) void mla_decode_stream_kernel(const DecodeParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kStages * kTileBytes];
  // pair exchange: softmax numerators (16 B per lane), per-head maxima and row sums
  __shared__ __attribute__((aligned(16))) u32x4 s_xp[kSWaves][64];
  __shared__ float s_xm[kSWaves][32];
  __shared__ float s_xr[kSWaves][32];  // per-head exponent references, for the waves that finalise other heads
  __shared__ int s_flag[kSWaves];
  // the CTA's range, staged once: per request r (= b - rb) its piece [t0, t1),
  // first stream tile, pieces and partial-slot offset; per stream tile its page id
  __shared__ int s_t0[kMaxCtaRequests], s_t1[kMaxCtaRequests], s_tbase[kMaxCtaRequests + 1];
  __shared__ int s_np[kMaxCtaRequests], s_slot0[kMaxCtaRequests];
  __shared__ int s_pid[2 * kMaxCtaBlocks];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hg = wave & 1;   // heads 32*hg .. +32 (two 16-head blocks hb)
  const int th = wave >> 1;  // tokens 16*th .. +16 of each tile for S; value dims 256*th .. +256 for O
  const int partner = wave ^ 2;
  const int g = lane >> 4;
  const int c = lane & 15;
  const int w = blockIdx.x;

  int rb, kb, re, ke;
  sload_i32x4(p.plan + 4 * w, rb, kb, re, ke);
  const int ps_mask = (1 << p.log2_ps) - 1;
  const int row_bytes = (int)(p.kv_row_stride * 2);
  const char* kv = reinterpret_cast<const char*>(p.kv);
  const uint32_t lds_ring = (uint32_t)(uintptr_t)(MLA_LDS char*)smem;

  // ---- per-lane LDS read offsets (bytes within a tile)
  const int xk = swz(c & 7);  // token 16*th + c has the swizzle of token c
  const int k_off_even = (16 * th + c) * kRowBytes + ((g ^ xk) << 4);
  const int k_off_odd = (16 * th + c) * kRowBytes + (((4 + g) ^ xk) << 4);
  int v_off[4];  // this wave's value half starts 512 bytes into the row (before swizzle groups)
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4)
    v_off[q4] = (4 * g + (c >> 2)) * kRowBytes + 256 * wave +
                ((2 * (q4 ^ (c >> 2)) + (((c & 3) >> 1) ^ (g & 1))) << 4) + ((c & 1) << 3);
  uint32_t dma_voff[kSDma];
#pragma unroll
  for (int k = 0; k < kSDma; ++k) {
    const int s = (wave + k * kSWaves) * 64 + lane;
    const int t = (s * 7282) >> 19;  // s / 72 for s < 2304
    dma_voff[k] = t * row_bytes + (((s - t * kRowChunks) ^ swz(t & 7)) << 4);
    // kept in an accumulation register (one move per use): otherwise the compiler recomputes the
    // offset (about ten vector instructions) at every tile for want of a free vector register
    asm volatile("" : "=a"(dma_voff[k]) : "0"(dma_voff[k]));
  }

  // ---- stage the range: request bounds, then one page id per 32-token tile
  int rlast = (ke == 0 ? re - 1 : re);
  rlast = min(rlast, p.batch - 1);
  const int nreq = min(rlast - rb + 1, kMaxCtaRequests);
  if (nreq <= 0) return;  // uniform: an empty range
  for (int r = threadIdx.x; r < nreq; r += 256) {
    const int b = rb + r;
    const int L = p.seq_lens[b];
    const int t0 = (r == 0) ? kb * kPlanBlock : 0;
    const int t1 = max(t0, (b == re) ? min(ke * kPlanBlock, L) : L);
    s_t0[r] = t0;
    s_t1[r] = t1;
    s_tbase[r + 1] = (t1 - t0 + kTile - 1) / kTile;
    const int first = p.plan[4 * p.num_ctas + 3 * b + 0];
    s_np[r] = p.plan[4 * p.num_ctas + 3 * b + 1];
    s_slot0[r] = p.plan[4 * p.num_ctas + 3 * b + 2] - first;
  }
  __syncthreads();
  if (wave == 0) {  // exclusive prefix of tile counts (64-wide scans)
    int carry = 0;
    for (int c0 = 0; c0 < nreq; c0 += 64) {
      const int r = c0 + lane;
      int v = r < nreq ? s_tbase[r + 1] : 0;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(v, o);
        if (lane >= o) v += u;
      }
      if (r < nreq) s_tbase[r + 1] = carry + v;
      carry += __shfl(v, 63);
    }
    if (lane == 0) s_tbase[0] = 0;
  }
  __syncthreads();
  const int ntiles_cta = min(s_tbase[nreq], 2 * kMaxCtaBlocks);
  {
    constexpr int kPer = 2 * kMaxCtaBlocks / 256;
    int pid[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int k = threadIdx.x + 256 * u;
      pid[u] = 0;
      if (k < ntiles_cta) {
        int lo = 0, hi = nreq - 1;  // last request whose first tile is <= k
        while (lo < hi) {
          const int mid = (lo + hi + 1) >> 1;
          if (s_tbase[mid] <= k) lo = mid;
          else hi = mid - 1;
        }
        const int t = s_t0[lo] + kTile * (k - s_tbase[lo]);
        pid[u] = p.page_table[(int64_t)(rb + lo) * p.pt_stride + (t >> p.log2_ps)];
      }
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int k = threadIdx.x + 256 * u;
      if (k < ntiles_cta) s_pid[k] = min(max(pid[u], 0), p.num_pages - 1);
    }
  }
  __syncthreads();

  // ---- stream cursors over (request, tile); all values wave-uniform
  auto seek = [&](Cursor& cur, int r) -> bool {  // first non-empty piece at or after request rb + r
    for (; r < nreq; ++r) {
      const int t0 = __builtin_amdgcn_readfirstlane(s_t0[r]);
      const int t1 = __builtin_amdgcn_readfirstlane(s_t1[r]);
      if (t1 > t0) {
        cur = Cursor{r, t0, t0, t1, 0};
        return true;
      }
    }
    return false;
  };
  auto advance = [&](Cursor& cur) -> bool {
    if (cur.q < 2) {
      ++cur.q;
      return true;
    }
    cur.t += kTile;
    return cur.t < cur.t1 ? true : seek(cur, cur.r + 1);
  };
  int iss_kv = 0;  // KV tiles issued (index into s_pid)
  auto issue = [&](const Cursor& cur, int n) {  // DMA stream tile n (at cur) into ring stage n % kStages
    const uint32_t lds_stage = lds_ring + (n % kStages) * kTileBytes;
    if (cur.q < 2) {  // query rows 32q .. +32 of request rb + r, staged like KV rows
      const int qrow_bytes = (int)(p.q_stride_h * 2);
      const char* qsrc = reinterpret_cast<const char*>(p.q) + ((int64_t)(rb + cur.r) * p.q_stride_b +
                                                             (int64_t)(32 * cur.q) * p.q_stride_h) * 2;
      // lane index from a volatile asm, so that these offsets are computed here and not kept in
      // registers across the loop
      int ln;
      asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
#pragma unroll
      for (int k = 0; k < kSDma; ++k) {
        const int s = (wave + k * kSWaves) * 64 + ln;
        const int t = (s * 7282) >> 19;  // s / 72
        const uint32_t voff = t * qrow_bytes + (((s - t * kRowChunks) ^ swz(t & 7)) << 4);
        dma16_saddr(qsrc, voff, lds_stage + (wave + k * kSWaves) * 1024);
      }
      return;
    }
    const int pid = __builtin_amdgcn_readfirstlane(s_pid[min(iss_kv++, 2 * kMaxCtaBlocks - 1)]);
    const char* tsrc = kv + ((int64_t)pid * (ps_mask + 1) + (cur.t & ps_mask)) * row_bytes;
    const int tlim = cur.t1 - 1 - cur.t;  // loads clamp to the piece's last token
    if (tlim >= kTile - 1) {
#pragma unroll
      for (int k = 0; k < kSDma; ++k) dma16_saddr(tsrc, dma_voff[k], lds_stage + (wave + k * kSWaves) * 1024);
    } else {
#pragma unroll
      for (int k = 0; k < kSDma; ++k) {
        const int s = (wave + k * kSWaves) * 64 + lane;
        const int t = (s * 7282) >> 19;
        const uint32_t voff = min(t, tlim) * row_bytes + (((s - t * kRowChunks) ^ swz(t & 7)) << 4);
        dma16_saddr(tsrc, voff, lds_stage + (wave + k * kSWaves) * 1024);
      }
    }
  };

  Cursor comp;
  if (!seek(comp, 0)) return;  // uniform: every piece of the range is empty
  Cursor iss = comp;

  // ---- queries of the current piece: qf[hb][ks] = head 32hg+16hb+c, dims 32ks + 8g .. +8, read from
  // the piece's query tile hg
  bf16x8 qf[2][18];

  int n_issued = 0;
  bool iss_valid = true;
  auto prologue = [&]() {
    for (int s = 0; s < kStages - 1 && iss_valid; ++s) {
      issue(iss, n_issued++);
      iss_valid = advance(iss);
    }
  };
  prologue();

  // ---- piece state; m_max and overflow are tracked per lane and reduced when needed
  f32x4 O[4][8];  // O^T of head block 0..3 (16 heads each), this wave's 8 dim blocks
  float m_ref[2] = {0.f, 0.f}, m_max[2], l_run[2];
  bool overflow = false;
  int attempt = 0;
  bool piece_start = true;
  Cursor piece_cur = comp;  // first KV tile of the piece (set when the stream reaches it)
  int piece_j = 0, piece_kv = 0, comp_kv = 0;  // stream / KV tile indices of it; KV tiles computed
  int st1 = 0, st2 = 0, st3 = 0;  // output stores issued 1, 2 and 3 iterations ago

  for (int j = 0;;) {
    if (comp.q < 2) {
      // a piece starts: its two query tiles (stream tiles j, j + 1). Wave (hg, th) takes the queries
      // of head group hg from tile j + hg once both have landed; the stage of tile j is refilled by
      // the DMA issued right after, so a barrier separates every wave's reads from that issue.
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        wait_vmcnt_dyn(kSDma * (n_issued - 1 - j) + st1 + st2 + st3);
        barrier_lds();
        st3 = st2;
        st2 = st1;
        st1 = 0;
        if (qt == 1) {
          const MLA_LDS char* QT = (const MLA_LDS char*)smem + ((j - 1 + hg) % kStages) * kTileBytes;
#pragma unroll
          for (int hb = 0; hb < 2; ++hb)
#pragma unroll
            for (int ks = 0; ks < 18; ++ks) {
              const int off =
                  ((ks & 1) ? k_off_odd : k_off_even) + 128 * (ks >> 1) + (16 * hb - 16 * th) * kRowBytes;
              qf[hb][ks] = *reinterpret_cast<const MLA_LDS bf16x8*>(QT + off);
            }
          // every wave's reads of tile j - 1 complete before any wave's next DMA overwrites its stage
          barrier_lds();
        }
        if (iss_valid) {
          issue(iss, n_issued++);
          iss_valid = advance(iss);
        }
        ++j;
        advance(comp);
      }
      piece_cur = comp;  // the piece's first KV tile
      piece_j = j;
      piece_kv = comp_kv;
    }
    // tile j's DMA is complete once at most (loads issued after it + stores since) remain
    wait_vmcnt_dyn(kSDma * (n_issued - 1 - j) + st1 + st2 + st3);
    barrier_lds();
    st3 = st2;
    st2 = st1;
    st1 = 0;
    if (iss_valid) {
      issue(iss, n_issued++);
      iss_valid = advance(iss);
    }
    if (piece_start) {
#pragma unroll
      for (int hq = 0; hq < 4; ++hq) {
#pragma unroll
        for (int db = 0; db < 8; ++db) O[hq][db] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
      l_run[0] = l_run[1] = 0.f;
      m_max[0] = m_max[1] = -INFINITY;
      overflow = false;
    }

    const MLA_LDS char* T = (const MLA_LDS char*)smem + (j % kStages) * kTileBytes;

    // ---- S^T[16 tokens x 16 heads] per head block hb, two accumulation chains each
    auto kread = [&](int ks) {
      const int off = ((ks & 1) ? k_off_odd : k_off_even) + 128 * (ks >> 1);
      return *reinterpret_cast<const MLA_LDS bf16x8*>(T + off);
    };
    f32x4 sacc[2][2];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) sacc[hb][0] = sacc[hb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 kbuf[kSKPrefetch];
#pragma unroll
    for (int r = 0; r < kSKPrefetch; ++r) kbuf[r] = kread(r);
#pragma unroll
    for (int ks = 0; ks < 18; ++ks) {
      const bf16x8 a = kbuf[ks % kSKPrefetch];
      if (ks + kSKPrefetch < 18) kbuf[ks % kSKPrefetch] = kread(ks + kSKPrefetch);
      sacc[0][ks & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[0][ks], sacc[0][ks & 1], 0, 0, 0);
      sacc[1][ks & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[1][ks], sacc[1][ks & 1], 0, 0, 0);
    }

    auto vread = [&](int db, int half) {
      const int off = v_off[db & 3] + 128 * (db >> 2) + half * 16 * kRowBytes;
      return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MLA_LDS bf16x4*)(T + off));
    };
    bf16x4 vlo[kSVPrefetch], vhi[kSVPrefetch];
#pragma unroll
    for (int r = 0; r < kSVPrefetch; ++r) {
      vlo[r] = vread(r, 0);
      vhi[r] = vread(r, 1);
    }

    // ---- softmax numerators of this wave's tokens: lane (g, c) holds tokens 16th + 4g + i of head c
    const int valid = comp.t1 - comp.t;  // tokens of this tile inside the piece
    float x[2][4], mt[2];                // mt: this lane's max over its 4 tokens
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const f32x4 sv = sacc[hb][0] + sacc[hb][1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[hb][i] = sv[i] * p.scale_log2;
        if (valid < kTile && 16 * th + 4 * g + i >= valid) x[hb][i] = -INFINITY;
      }
      mt[hb] = fmaxf(fmaxf(x[hb][0], x[hb][1]), fmaxf(x[hb][2], x[hb][3]));
    }
    if (piece_start && attempt == 0) {
      // exponent reference: max over the first tile's 32 tokens, agreed with the partner
      const float w0 = wave_max_g(mt[0]), w1 = wave_max_g(mt[1]);
      if (g == 0) {
        s_xm[wave][c] = w0;
        s_xm[wave][16 + c] = w1;
      }
      barrier_lds();
      m_ref[0] = fmaxf(w0, s_xm[partner][c]);
      m_ref[1] = fmaxf(w1, s_xm[partner][16 + c]);
    }
    u32x2 pown[2];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      m_max[hb] = fmaxf(m_max[hb], mt[hb]);
      overflow |= mt[hb] > m_ref[hb] + kSOverflowLog2;
      float pr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[i] = __builtin_amdgcn_exp2f(x[hb][i] - m_ref[hb]);
        l_run[hb] += pr[i];
      }
      pown[hb][0] = pack_bf16x2(pr[0], pr[1]);
      pown[hb][1] = pack_bf16x2(pr[2], pr[3]);
    }
    // P^T B operand of lane (g, c): k = 8g + i is token 4g + i (i < 4, half 0) or 16 + 4g + i - 4 (half 1)
    s_xp[wave][lane] = u32x4{pown[0][0], pown[0][1], pown[1][0], pown[1][1]};
    barrier_lds();
    // P^T B operands of all 64 heads: head block 2 hg' + hb takes tokens 0..15 from wave hg' and
    // tokens 16..31 from wave hg' + 2
    bf16x8 pb[4];
#pragma unroll
    for (int hgi = 0; hgi < 2; ++hgi) {
      const u32x4 p0 = s_xp[hgi][lane], p1 = s_xp[hgi + 2][lane];
      pb[2 * hgi + 0] = __builtin_bit_cast(bf16x8, (u32x4{p0[0], p0[1], p1[0], p1[1]}));
      pb[2 * hgi + 1] = __builtin_bit_cast(bf16x8, (u32x4{p0[2], p0[3], p1[2], p1[3]}));
    }

    // ---- O^T[16 dims x 16 heads] += V^T . P^T: this wave's 8 dim blocks, all 4 head blocks (every
    // staged V row is read by one wave)
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const bf16x8 a =
          __builtin_shufflevector(vlo[db % kSVPrefetch], vhi[db % kSVPrefetch], 0, 1, 2, 3, 4, 5, 6, 7);
      if (db + kSVPrefetch < 8) {
        vlo[db % kSVPrefetch] = vread(db + kSVPrefetch, 0);
        vhi[db % kSVPrefetch] = vread(db + kSVPrefetch, 1);
      }
#pragma unroll
      for (int hq = 0; hq < 4; ++hq) O[hq][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[hq], O[hq][db], 0, 0, 0);
    }

    const bool piece_end = comp.t + kTile >= comp.t1;
    piece_start = false;
    if (piece_end) {
      // CTA-wide overflow vote; the row sums of the pair travel with it
      const float lw0 = wave_sum_g(l_run[0]), lw1 = wave_sum_g(l_run[1]);
      if (g == 0) {
        s_xm[wave][c] = lw0;
        s_xm[wave][16 + c] = lw1;
        s_xr[wave][c] = m_ref[0];
        s_xr[wave][16 + c] = m_ref[1];
      }
      const bool wave_overflow = __ballot(overflow) != 0;
      if (lane == 0) s_flag[wave] = wave_overflow ? 1 : 0;
      barrier_lds();
      const bool any_overflow = (s_flag[0] | s_flag[1] | s_flag[2] | s_flag[3]) != 0;
      if (any_overflow && attempt == 0) {
        // rare: rewind the stream to the piece start and rerun it with the exact max of the pair
        wait_vmcnt<0>();
        barrier_lds();
        const float w0 = wave_max_g(m_max[0]), w1 = wave_max_g(m_max[1]);
        if (g == 0) {
          s_xm[wave][c] = w0;
          s_xm[wave][16 + c] = w1;
        }
        barrier_lds();
        m_ref[0] = fmaxf(w0, s_xm[partner][c]);
        m_ref[1] = fmaxf(w1, s_xm[partner][16 + c]);
        comp = piece_cur;
        iss = piece_cur;
        j = piece_j;
        n_issued = piece_j;
        iss_kv = piece_kv;
        comp_kv = piece_kv;
        iss_valid = true;
        st1 = st2 = st3 = 0;
        attempt = 1;
        piece_start = true;
        prologue();
        continue;
      }
      attempt = 0;
      // every wave holds all 64 heads' outputs for its dims: row sums (both token halves) and
      // exponent references of head block 2 hg' + hb come from waves hg' and hg' + 2
      float l_tot[4], m_all[4];
#pragma unroll
      for (int hq = 0; hq < 4; ++hq) {
        const int src = hq >> 1, hx = 16 * (hq & 1) + c;
        l_tot[hq] = s_xm[src][hx] + s_xm[src + 2][hx];
        m_all[hq] = s_xr[src][hx];
      }

      // ---- finalise: lane holds heads 16hq+c, dims 128wave + 16db + 4g + (0..3); wave w writes the
      // LSE of head block w
      const int b = rb + comp.r;
      const int npieces = __builtin_amdgcn_readfirstlane(s_np[comp.r]);
      int stores = 0;
#pragma unroll
      for (int hq = 0; hq < 4; ++hq) {
        const int h = 16 * hq + c;
        const float inv = l_tot[hq] > 0.f ? 1.f / l_tot[hq] : 0.f;
        const float lse_nat =
            l_tot[hq] > 0.f ? (m_all[hq] + log2f(l_tot[hq])) * 0.69314718055994531f : -INFINITY;
        if (npieces == 1) {
          __bf16* orow = p.out + (int64_t)b * p.out_stride_b + (int64_t)h * p.out_stride_h + 128 * wave + 4 * g;
#pragma unroll
          for (int db = 0; db < 8; ++db) {
            u32x2 v;
            v[0] = pack_bf16x2(O[hq][db][0] * inv, O[hq][db][1] * inv);
            v[1] = pack_bf16x2(O[hq][db][2] * inv, O[hq][db][3] * inv);
            *reinterpret_cast<u32x2*>(orow + 16 * db) = v;
          }
          stores += 8;
          if (p.lse != nullptr && hq == wave) {
            if (g == 0) p.lse[(int64_t)b * p.lse_stride_b + h] = lse_nat;
            stores += 1;
          }
        } else {
          const int slot = __builtin_amdgcn_readfirstlane(s_slot0[comp.r]) + w;
          if (slot >= 0 && slot < p.ws_slots) {
            __bf16* orow = p.ws_o + ((int64_t)slot * p.heads + h) * kVDim + 128 * wave + 4 * g;
#pragma unroll
            for (int db = 0; db < 8; ++db) {
              u32x2 v;
              v[0] = pack_bf16x2(O[hq][db][0] * inv, O[hq][db][1] * inv);
              v[1] = pack_bf16x2(O[hq][db][2] * inv, O[hq][db][3] * inv);
              *reinterpret_cast<u32x2*>(orow + 16 * db) = v;
            }
            stores += 8;
            if (hq == wave) {
              if (g == 0) p.ws_lse[(int64_t)slot * p.heads + h] = lse_nat;
              stores += 1;
            }
          }
        }
      }
      st1 = stores;
    }

    ++j;
    ++comp_kv;
    if (!advance(comp)) break;
    if (piece_end) piece_start = true;
  }
}

}  // namespace

hipError_t launch_decode_stream(const DecodeParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(mla_decode_stream_kernel, dim3(p.num_ctas), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mla
