// Warp-specialized absorbed-MLA decode for 64 query heads and pages of >= 32 tokens (the Kimi-K2 /
// DeepSeek-V3 decode shape on one GPU). Same plan, workspace and outputs as mla_decode_kernel.
//
//  * The CTA's whole (request, token) range is one stream of 32-row tiles: per piece, two tiles of
//    queries (heads 0..31, 32..63; a query row has the latent row's 576 dims, so it is staged like
//    a KV row) and then the piece's 32-token KV tiles, through a 4-stage LDS ring filled by
//    global->LDS DMA (non-temporal for the KV rows, which are read once). The page id of every KV
//    tile and the bounds of every request of the range are staged in LDS once, at CTA start.
//  * 8 waves, two per SIMD, in two roles that run one tile apart:
//      score waves (hg, th) = (s & 1, s >> 1), s = 0..3 (heads 32hg .. 32hg+31, tokens 16th .. +16
//      of a tile):
//        S^T[16 tokens x 32 heads] = K . Q^T                  36 MFMAs, 18 K reads
//        softmax numerators against the piece's reference (its first tile's max over both halves,
//        agreed by the pair (hg, 0) / (hg, 1) at the piece's first KV tile), written as bf16 to a
//        double-buffered P block in LDS
//      output waves o = 0..3 (value dims 128o .. 128o+127, all 64 heads), one tile behind:
//        O^T[128 dims x 64 heads] += V^T . P^T                 32 MFMAs, 16 transposing V reads
//    Every K row is read from LDS by two waves, every V row by one. A SIMD holds one wave of each
//    role, so one role's LDS and barrier waits are covered by the other's MFMAs. One barrier per step
//    (two at a piece's first KV tile): step j scores tile j and accumulates tile j - 1; the output
//    waves normalise and store a piece (bf16 output, or the bf16 partial of a split request) and
//    write its LSE.
//  * No accumulator rescaling: exponents are taken against the piece's first-tile max; a piece whose
//    later scores exceed it by 2^64 is rerun with its exact max (the vote is taken at the step after
//    the piece's last tile, before any wave touches the next tile).
//  * Barriers wait on LDS only; each wave counts its own DMA loads and output stores and waits with
//    an exact vmcnt.
#include <type_traits>

#include "mla_common.h"
#include "mla_device.h"

namespace mla {
namespace {

constexpr int kWWaves = 8;
constexpr int kWAhead = 2;         // stream tiles in flight beyond the one being scored
// A tile's 36 wave-wide DMA loads ("parts") are split between the roles: score wave r issues parts
// r + 4k (k < kWScoreParts), output wave r parts 4 kWScoreParts + r + 4k (k < kWOutParts); a role
// issues its parts after its step's work (instead of right after the step's barrier)
// when its Late flag is set.
constexpr int kWScoreParts = 0;
constexpr int kWOutParts = 9;
constexpr bool kWScoreLate = false;
constexpr bool kWOutLate = false;
static_assert(4 * (kWScoreParts + kWOutParts) == kTileDma, "every part of a tile is issued once");
constexpr int kWKPrefetch = 6;     // K operands in flight
constexpr int kWVPrefetch = 4;     // V operand pairs in flight
constexpr int kWMaxTiles = 2 * kMaxCtaBlocks;
constexpr float kWOverflowLog2 = 64.0f;

struct WCursor {
  int r, t, t0, t1, q;  // request rb + r, piece [t0, t1); q < 2: query tile q, q == 2: KV tile at token t
};

// kSmall: pages of fewer than 32 tokens. A tile's rows then lie on several pages, so instead of one
// page id per tile the DMA takes one 32-bit row offset (from the pool base) per token: score wave 0
// loads the page-table entries of stream tile n at step n - 4, writes the tile's 32 row offsets to
// slot n % 4 of a ring in LDS at step n - 3, and the output waves read them at step n - 2, after that
// step's barrier, when they issue the tile. The launcher takes this path only when every row offset
// of the pool fits in 32 bits.
//
// kLoop: the launch has fewer CTAs than the plan has ranges (a plan laid out for a larger grid, as a
// captured decode step's is); CTA b then runs ranges b, b + gridDim.x, ... in turn and stops at the
// first padding range. Without it (at most one range per compute unit) each CTA runs range blockIdx.x
// and the body has no loop around it: the loop makes the compiler keep values across both roles'
// step loops and spill.
template <bool kSmall, bool kLoop>
__global__ __launch_bounds__(kWWaves * 64, 1) void mla_decode_ws_kernel(const DecodeParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kStages * kTileBytes];
  // softmax numerators of the last two scored tiles: [tile parity][head block][lane], 16 B per lane
  __shared__ __attribute__((aligned(16))) u32x4 s_p[2][4][64];
  __shared__ float s_l[2][64];   // per token half and head: row sums of the piece that just ended
  __shared__ float s_mref[64];   // per head: that piece's exponent reference
  __shared__ float s_mx[2][64];  // per token half and head: a max (piece start: first tile; end: piece)
  __shared__ int s_flag[4];      // per score wave: that piece overflowed its exponent reference
  __shared__ int s_t0[kMaxCtaRequests], s_t1[kMaxCtaRequests], s_tbase[kMaxCtaRequests + 1];
  __shared__ int s_np[kMaxCtaRequests], s_slot0[kMaxCtaRequests];
  __shared__ int s_pid[kWMaxTiles];  // page id per KV tile; kSmall: the row-offset ring [4][32]

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool scorer = wave < 4;
  const int role = wave & 3;  // score wave: head block; output wave: value-dim quarter

  // Plan range w; false for a padding range (all later ranges are padding too).
  auto range = [&](const int w) -> bool {
    // the lane index from a volatile asm: what derives from it is computed per range, not hoisted
    // out of a loop over ranges
    int lane;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
    const int g = lane >> 4;
    const int c = lane & 15;
    int rb, kb, re, ke;
    sload_i32x4(p.plan + 4 * w, rb, kb, re, ke);
    if (rb >= p.batch) return false;
    const int ps_mask = (1 << p.log2_ps) - 1;
    const int row_bytes = (int)(p.kv_row_stride * 2);
    const char* kv = reinterpret_cast<const char*>(p.kv);
    const uint32_t lds_ring = (uint32_t)(uintptr_t)(MLA_LDS char*)smem;

    // ---- per-lane LDS read offsets (bytes within a tile)
    const int xk = swz(c & 7);  // token 16 tb + c has the swizzle of token c
    const int k_off_even = c * kRowBytes + ((g ^ xk) << 4);
    const int k_off_odd = c * kRowBytes + (((4 + g) ^ xk) << 4);
    int v_off[4];  // output wave `role`: value dims 128 role .. +128 start 256 role bytes into the row
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      v_off[q4] = (4 * g + (c >> 2)) * kRowBytes + 256 * role +
                  ((2 * (q4 ^ (c >> 2)) + (((c & 3) >> 1) ^ (g & 1))) << 4) + ((c & 1) << 3);
    // DMA: wave-wide load `part` of a tile covers slots 64 part + lane (token slot / 72, chunk slot % 72
    // at its swizzled position); wave w issues parts w, w + 8, ... (score waves 5, output waves 4)

    // ---- stage the range: request bounds, then one page id per 32-token tile
    int rlast = (ke == 0 ? re - 1 : re);
    rlast = min(rlast, p.batch - 1);
    const int nreq = min(rlast - rb + 1, kMaxCtaRequests);
    if (nreq <= 0) return true;  // uniform: an empty range
    // The first piece is request rb's in all but rare cases (rb's part of the range is empty only for
    // an empty request): the output waves load its two query tiles into ring stages 0 and 1 now, so
    // that they land while the range is staged (the staging's barriers wait on LDS only). If the
    // first piece turns out to be another request's, the stream issues its query tiles into the same
    // stages after these loads, and loads of one wave complete in order.
    constexpr int kEarlyQueryDma = 2 * kWOutParts;
    if (!scorer) {
      const int qrow_bytes = (int)(p.q_stride_h * 2);
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const char* qsrc = reinterpret_cast<const char*>(p.q) +
                           ((int64_t)rb * p.q_stride_b + (int64_t)(32 * qt) * p.q_stride_h) * 2;
#pragma unroll
        for (int k = 0; k < kWOutParts; ++k) {
          const int part = 4 * kWScoreParts + role + 4 * k;
          const int s = part * 64 + lane;
          const int t = (s * 7282) >> 19;  // s / 72
          dma16_saddr(qsrc, t * qrow_bytes + (((s - t * kRowChunks) ^ swz(t & 7)) << 4),
                      lds_ring + qt * kTileBytes + part * 1024);
        }
      }
    }
    for (int r = threadIdx.x; r < nreq; r += kWWaves * 64) {
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
    barrier_lds();
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
    barrier_lds();
    const int ntiles_cta = min(s_tbase[nreq], kWMaxTiles);
    if constexpr (!kSmall) {
      constexpr int kPer = kWMaxTiles / (kWWaves * 64);
      int pid[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int k = threadIdx.x + kWWaves * 64 * u;
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
        const int k = threadIdx.x + kWWaves * 64 * u;
        if (k < ntiles_cta) s_pid[k] = min(max(pid[u], 0), p.num_pages - 1);
      }
    }
    barrier_lds();

    // ---- stream cursors over (request, tile); all values wave-uniform
    auto seek = [&](WCursor& cur, int r) -> bool {  // first non-empty piece at or after request rb + r
      for (; r < nreq; ++r) {
        const int t0 = __builtin_amdgcn_readfirstlane(s_t0[r]);
        const int t1 = __builtin_amdgcn_readfirstlane(s_t1[r]);
        if (t1 > t0) {
          cur = WCursor{r, t0, t0, t1, 0};
          return true;
        }
      }
      return false;
    };
    auto advance = [&](WCursor& cur) -> bool {
      if (cur.q < 2) {
        ++cur.q;
        return true;
      }
      cur.t += kTile;
      return cur.t < cur.t1 ? true : seek(cur, cur.r + 1);
    };
    // Each role runs its own copy of the step loop (the same stream, the same barriers), so that only
    // that role's state is live in its registers.
    auto run = [&](auto role_tag) {
    constexpr bool kScore = decltype(role_tag)::value;
    constexpr int nparts = kScore ? kWScoreParts : kWOutParts;
    const int part0 = kScore ? role : 4 * kWScoreParts + role;  // this wave's parts: part0 + 4k
    uint32_t dma_voff[nparts > 0 ? nparts : 1];
#pragma unroll
    for (int k = 0; k < nparts; ++k) {
      const int s = (part0 + 4 * k) * 64 + lane;
      const int t = (s * 7282) >> 19;  // s / 72 for s < 2304
      const int chunk_off = ((s - t * kRowChunks) ^ swz(t & 7)) << 4;
      dma_voff[k] = kSmall ? (t << 16) | chunk_off : t * row_bytes + chunk_off;
    }
    int iss_kv = 0;  // KV tiles issued (index into s_pid)
    // vector-memory operations this wave issued, and the count right after its parts of stream tile n
    // (kept for n % 4): tile n has landed once at most (ops - mark) operations are outstanding
    int ops = kScore ? 0 : kEarlyQueryDma, mark0 = kScore ? 0 : kWOutParts, mark1 = ops, mark2 = 0, mark3 = 0;
    auto issue = [&](const WCursor& cur, int n) {  // this wave's DMA parts of stream tile n (at cur)
      const uint32_t stage = lds_ring + (n % kStages) * kTileBytes;
      if (cur.q < 2) {  // query rows 32q .. +32 of request rb + r
        const int qrow_bytes = (int)(p.q_stride_h * 2);
        const char* qsrc = reinterpret_cast<const char*>(p.q) +
                           ((int64_t)(rb + cur.r) * p.q_stride_b + (int64_t)(32 * cur.q) * p.q_stride_h) * 2;
        int ln;  // lane index from a volatile asm, so these offsets are computed here
        asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
#pragma unroll
        for (int k = 0; k < nparts; ++k) {
          const int s = (part0 + 4 * k) * 64 + ln;
          const int t = (s * 7282) >> 19;
          dma16_saddr(qsrc, t * qrow_bytes + (((s - t * kRowChunks) ^ swz(t & 7)) << 4),
                      stage + (part0 + 4 * k) * 1024);
        }
      } else if constexpr (kSmall) {  // each lane's token row from the offset ring (clamped rows included)
        const int ring = (n & 3) * 32;
#pragma unroll
        for (int k = 0; k < nparts; ++k)
          dma16_saddr_nt(kv, (uint32_t)s_pid[ring + (dma_voff[k] >> 16)] + (dma_voff[k] & 0xffff),
                         stage + (part0 + 4 * k) * 1024);
      } else {
        const int pid = __builtin_amdgcn_readfirstlane(s_pid[min(iss_kv++, kWMaxTiles - 1)]);
        const char* tsrc = kv + ((int64_t)pid * (ps_mask + 1) + (cur.t & ps_mask)) * row_bytes;
        const int tlim = cur.t1 - 1 - cur.t;  // loads clamp to the piece's last token
        if (tlim >= kTile - 1) {
#pragma unroll
          for (int k = 0; k < nparts; ++k) dma16_saddr_nt(tsrc, dma_voff[k], stage + (part0 + 4 * k) * 1024);
        } else {
          int ln;
          asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
#pragma unroll
          for (int k = 0; k < nparts; ++k) {
            const int s = (part0 + 4 * k) * 64 + ln;
            const int t = (s * 7282) >> 19;
            dma16_saddr_nt(tsrc, min(t, tlim) * row_bytes + (((s - t * kRowChunks) ^ swz(t & 7)) << 4),
                           stage + (part0 + 4 * k) * 1024);
          }
        }
      }
      ops += nparts;
      const int m = n & 3;
      mark0 = m == 0 ? ops : mark0;
      mark1 = m == 1 ? ops : mark1;
      mark2 = m == 2 ? ops : mark2;
      mark3 = m == 3 ? ops : mark3;
    };

    WCursor cs;  // the tile scored at this step
    if (!seek(cs, 0)) {  // uniform: every piece of the range is empty (no barrier follows)
      wait_vmcnt<0>();   // the early query loads land before the CTA can end
      return;
    }
    WCursor iss = cs;
    int n_issued = 0;
    bool iss_valid = true;
    if constexpr (nparts > 0) {
      if (cs.r == 0) {  // the early query loads are stream tiles 0 and 1 (a piece starts at q = 0)
        for (int s = 0; s < 2 && iss_valid; ++s) {
          ++n_issued;
          iss_valid = advance(iss);
        }
      } else {  // request rb is empty: its query loads land before the stream reuses their stages
        wait_vmcnt<0>();
        ops = mark0 = mark1 = 0;
      }
    }
    auto prologue = [&](const int from) {
      if constexpr (nparts == 0) return;  // a role without DMA parts keeps no issue cursor
      for (int s = from; s < kWAhead && iss_valid; ++s) {
        issue(iss, n_issued++);
        iss_valid = advance(iss);
      }
    };
    // kSmall: score wave 0's row-offset producer. la is the stream tile (index la_n) whose
    // page-table entries are in flight; lane l (< 32) holds its token t + l, clamped to the piece.
    WCursor la = cs;
    int la_n = 0, la_tok = 0, la_page = 0;
    bool la_valid = false, la_kv = false;
    auto la_load = [&]() {
      la_kv = la_valid && la.q == 2;
      if (la_kv) {
        la_tok = min(la.t + (lane & 31), la.t1 - 1);
        la_page = p.page_table[(int64_t)(rb + la.r) * p.pt_stride + (la_tok >> p.log2_ps)];
      }
    };
    auto la_store = [&]() {  // waits for la_page (this wave issues no other vector-memory loads)
      if (la_kv && lane < 32) {
        const uint32_t page = (uint32_t)min(max(la_page, 0), p.num_pages - 1);
        s_pid[(la_n & 3) * 32 + lane] = (int)(((page << p.log2_ps) | (uint32_t)(la_tok & ps_mask)) * (uint32_t)row_bytes);
      }
    };
    auto la_step = [&]() {  // store the in-flight tile's offsets, then load the next tile's entries
      la_store();
      if (la_valid) la_valid = advance(la);
      ++la_n;
      la_load();
    };
    auto seed = [&](const WCursor& from, int n0) {  // offsets of tiles n0 .. n0 + 2; n0 + 3 in flight
      la = from;
      la_valid = true;
      int tok[3], pg[3];
      bool kv3[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) {  // the three tiles' page-table loads back to back
        kv3[i] = la_valid && la.q == 2;
        tok[i] = min(la.t + (lane & 31), la.t1 - 1);
        pg[i] = kv3[i] ? p.page_table[(int64_t)(rb + la.r) * p.pt_stride + (tok[i] >> p.log2_ps)] : 0;
        if (la_valid) la_valid = advance(la);
      }
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        if (kv3[i] && lane < 32) {
          const uint32_t page = (uint32_t)min(max(pg[i], 0), p.num_pages - 1);
          s_pid[((n0 + i) & 3) * 32 + lane] =
              (int)(((page << p.log2_ps) | (uint32_t)(tok[i] & ps_mask)) * (uint32_t)row_bytes);
        }
      }
      la_n = n0 + 3;
      la_load();
    };
    if constexpr (kSmall) {  // every wave: the first tiles' offsets before the first DMA
      if constexpr (kScore) if (role == 0) seed(cs, 0);
      barrier_lds();
    }
    prologue(n_issued);

    // score-wave state: queries of head blocks 2 hg, 2 hg + 1; per head block (lane: head c of it)
    // the piece's reference, max and this half's row sum
    const int hg = role & 1, th = role >> 1;
    bf16x8 qf[2][18];
    float m_ref[2] = {0.f, 0.f}, m_max[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
    bool overflow = false, first_kv = true;
    // output-wave state
    f32x4 O[4][8];
#pragma unroll
    for (int hq = 0; hq < 4; ++hq)
#pragma unroll
      for (int db = 0; db < 8; ++db) O[hq][db] = f32x4{0.f, 0.f, 0.f, 0.f};

    int attempt = 0;
    bool s_valid = true;                          // cs is a tile
    bool prev_kv = false, prev_end = false;       // the tile scored at the previous step
    int prev_r = 0;
    WCursor piece_cur = cs;                       // first KV tile of the current piece
    int piece_j = 0, piece_kv = 0, comp_kv = 0;   // its stream / KV indices; KV tiles scored

    for (int j = 0;;) {
      // ---- step j: tile j (cs) lands; wait for this wave's DMA parts of it, then the whole CTA's
      if (j < n_issued) {
        const int m = j & 3;
        wait_vmcnt_dyn(ops - (m == 0 ? mark0 : m == 1 ? mark1 : m == 2 ? mark2 : mark3));
      }
      barrier_lds();

      if (prev_kv && prev_end && attempt == 0 && (s_flag[0] | s_flag[1] | s_flag[2] | s_flag[3]) != 0) {
        // rare: the piece that just ended overflowed its exponent reference somewhere. Drain, rewind
        // the stream to its first KV tile and rerun it with each head's exact max (queries are still
        // in registers: no wave has touched tile j yet).
        wait_vmcnt<0>();
        barrier_lds();
        if constexpr (kScore) {
#pragma unroll
          for (int hb = 0; hb < 2; ++hb) {  // the piece's exact max over both token halves
            const int h = 32 * hg + 16 * hb + c;
            m_ref[hb] = fmaxf(s_mx[0][h], s_mx[1][h]);
            m_max[hb] = -INFINITY;
            l_run[hb] = 0.f;
          }
          overflow = false;
        } else {
#pragma unroll
          for (int hq = 0; hq < 4; ++hq)
#pragma unroll
            for (int db = 0; db < 8; ++db) O[hq][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        attempt = 1;
        first_kv = true;
        cs = piece_cur;
        iss = piece_cur;
        j = piece_j;
        n_issued = nparts > 0 ? piece_j : 0;
        iss_kv = piece_kv;
        comp_kv = piece_kv;
        iss_valid = true;
        s_valid = true;
        prev_kv = false;
        ops = 0;
        if constexpr (kSmall) {  // the rewound tiles' offsets again (their ring slots were reused)
          if constexpr (kScore) if (role == 0) seed(piece_cur, piece_j);
          barrier_lds();
        }
        prologue(0);
        continue;
      }
      if (prev_kv && prev_end) attempt = 0;

      constexpr bool kLate = kScore ? kWScoreLate : kWOutLate;
      if (nparts > 0 && iss_valid && !kLate) {
        issue(iss, n_issued++);
        iss_valid = advance(iss);
      }

      const bool cur_kv = s_valid && cs.q == 2;
      const bool cur_end = cur_kv && cs.t + kTile >= cs.t1;
      if (cur_kv && first_kv) {
        piece_cur = cs;
        piece_j = j;
        piece_kv = comp_kv;
      }

      if constexpr (kScore) {
        const MLA_LDS char* T = (const MLA_LDS char*)smem + (j % kStages) * kTileBytes;
        if (s_valid && cs.q < 2) {
          // a piece starts: head group hg reads its 32 query rows (two head blocks) from query tile hg
          if (hg == cs.q) {
#pragma unroll
            for (int hb = 0; hb < 2; ++hb)
#pragma unroll
              for (int ks = 0; ks < 18; ++ks) {
                const int off = ((ks & 1) ? k_off_odd : k_off_even) + 128 * (ks >> 1) + 16 * hb * kRowBytes;
                qf[hb][ks] = *reinterpret_cast<const MLA_LDS bf16x8*>(T + off);
              }
          }
        } else if (cur_kv) {
          // ---- S^T[16 tokens (half th) x 16 heads] for head blocks hb = 0, 1; two chains each
          auto kread = [&](int ks) {
            const int off = ((ks & 1) ? k_off_odd : k_off_even) + 128 * (ks >> 1) + 16 * th * kRowBytes;
            return *reinterpret_cast<const MLA_LDS bf16x8*>(T + off);
          };
          f32x4 sacc[2][2];
#pragma unroll
          for (int hb = 0; hb < 2; ++hb) sacc[hb][0] = sacc[hb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
          bf16x8 kbuf[kWKPrefetch];
#pragma unroll
          for (int r = 0; r < kWKPrefetch; ++r) kbuf[r] = kread(r);
#pragma unroll
          for (int ks = 0; ks < 18; ++ks) {
            const bf16x8 a = kbuf[ks % kWKPrefetch];
            if (ks + kWKPrefetch < 18) kbuf[ks % kWKPrefetch] = kread(ks + kWKPrefetch);
            sacc[0][ks & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[0][ks], sacc[0][ks & 1], 0, 0, 0);
            sacc[1][ks & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[1][ks], sacc[1][ks & 1], 0, 0, 0);
          }
          // ---- softmax numerators: lane (g, c) holds head 32 hg + 16 hb + c, tokens 16 th + 4 g + i
          const int valid = cs.t1 - cs.t;
          float x[2][4], mt[2];
#pragma unroll
          for (int hb = 0; hb < 2; ++hb) {
            const f32x4 sv = sacc[hb][0] + sacc[hb][1];
            mt[hb] = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              x[hb][i] = sv[i] * p.scale_log2;
              if (valid < kTile && 16 * th + 4 * g + i >= valid) x[hb][i] = -INFINITY;
              mt[hb] = fmaxf(mt[hb], x[hb][i]);
            }
            mt[hb] = wave_max_g(mt[hb]);  // this head's max over this half of the tile
          }
          if (first_kv && attempt == 0) {
            // the piece's reference: the first tile's max over both halves, agreed with the wave that
            // holds the other half (an extra barrier, which every wave takes at this step; the output
            // waves are idle here, the previous tile being a query tile)
            if (g == 0) {
              s_mx[th][32 * hg + c] = mt[0];
              s_mx[th][32 * hg + 16 + c] = mt[1];
            }
            barrier_lds();
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
              const int h = 32 * hg + 16 * hb + c;
              m_ref[hb] = fmaxf(s_mx[0][h], s_mx[1][h]);
            }
          }
          u32x2 pown[2];
#pragma unroll
          for (int hb = 0; hb < 2; ++hb) {
            m_max[hb] = fmaxf(m_max[hb], mt[hb]);
            overflow |= mt[hb] > m_ref[hb] + kWOverflowLog2;
            float pr[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              pr[i] = __builtin_amdgcn_exp2f(x[hb][i] - m_ref[hb]);
              l_run[hb] += pr[i];
            }
            pown[hb][0] = pack_bf16x2(pr[0], pr[1]);
            pown[hb][1] = pack_bf16x2(pr[2], pr[3]);
          }
          // the P^T B operand of head block 2 hg + hb, lane (g, c): k = 8g + i is token 4g + i (i < 4,
          // written by half 0) or 16 + 4g + i - 4 (half 1)
#pragma unroll
          for (int hb = 0; hb < 2; ++hb)
            reinterpret_cast<u32x2*>(&s_p[j & 1][2 * hg + hb][lane])[th] = pown[hb];
          if (cur_end) {
            // publish this half's row sums, the reference, the max and the overflow; reset
            const bool wave_overflow = __ballot(overflow) != 0;
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
              const float l_half = wave_sum_g(l_run[hb]);
              const int h = 32 * hg + 16 * hb + c;
              if (g == 0) {
                s_l[th][h] = l_half;
                s_mx[th][h] = m_max[hb];
                if (th == 0) s_mref[h] = m_ref[hb];
              }
              m_max[hb] = -INFINITY;
              l_run[hb] = 0.f;
            }
            if (lane == 0) s_flag[role] = wave_overflow ? 1 : 0;
            overflow = false;
          }
        }
      } else {
        // the score waves' reference exchange at a piece's first KV tile takes a barrier: take it too
        // (the previous tile is the piece's second query tile, so there is no output work here)
        if (cur_kv && first_kv && attempt == 0) barrier_lds();
      }
      if constexpr (!kScore) if (prev_kv) {
        // ---- output wave: O^T[16 dims x 16 heads] += V^T . P^T for tile j - 1, this wave's 8 dim
        // blocks and all 4 head blocks
        const MLA_LDS char* T = (const MLA_LDS char*)smem + ((j - 1) % kStages) * kTileBytes;
        auto vread = [&](int db, int half) {
          const int off = v_off[db & 3] + 128 * (db >> 2) + half * 16 * kRowBytes;
          return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MLA_LDS bf16x4*)(T + off));
        };
        bf16x4 vlo[kWVPrefetch], vhi[kWVPrefetch];
#pragma unroll
        for (int r = 0; r < kWVPrefetch; ++r) {
          vlo[r] = vread(r, 0);
          vhi[r] = vread(r, 1);
        }
        bf16x8 pb[4];
#pragma unroll
        for (int hq = 0; hq < 4; ++hq) pb[hq] = __builtin_bit_cast(bf16x8, s_p[(j - 1) & 1][hq][lane]);
#pragma unroll
        for (int db = 0; db < 8; ++db) {
          const bf16x8 a =
              __builtin_shufflevector(vlo[db % kWVPrefetch], vhi[db % kWVPrefetch], 0, 1, 2, 3, 4, 5, 6, 7);
          if (db + kWVPrefetch < 8) {
            vlo[db % kWVPrefetch] = vread(db + kWVPrefetch, 0);
            vhi[db % kWVPrefetch] = vread(db + kWVPrefetch, 1);
          }
#pragma unroll
          for (int hq = 0; hq < 4; ++hq)
            O[hq][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[hq], O[hq][db], 0, 0, 0);
        }
        if (prev_end && (s_flag[0] | s_flag[1] | s_flag[2] | s_flag[3]) == 0) {
          // ---- the piece ended at tile j - 1: normalise and write this wave's dims of all 64 heads.
          // (An overflowed first attempt writes nothing; the vote at the next step reruns it.)
          const int b = rb + prev_r;
          const int npieces = __builtin_amdgcn_readfirstlane(s_np[prev_r]);
          const int slot = __builtin_amdgcn_readfirstlane(s_slot0[prev_r]) + w;
          const bool to_ws = npieces != 1;
          if (!to_ws || (slot >= 0 && slot < p.ws_slots)) {
#pragma unroll
            for (int hq = 0; hq < 4; ++hq) {
              const int h = 16 * hq + c;
              const float l = s_l[0][h] + s_l[1][h];
              const float inv = l > 0.f ? 1.f / l : 0.f;
              if (to_ws) {
                // bf16 partial for the merge, one 16-byte chunk per dim-block pair (2 pp, 2 pp + 1): chunk
                // 16 role + 4 pp + g of the row (the chunk order of mla_amd.h)
                __bf16* orow = p.ws_o + ((int64_t)slot * p.heads + h) * kVDim + 128 * role + 8 * g;
#pragma unroll
                for (int pp = 0; pp < 4; ++pp) {
                  u32x4 v;
                  v[0] = pack_bf16x2(O[hq][2 * pp][0] * inv, O[hq][2 * pp][1] * inv);
                  v[1] = pack_bf16x2(O[hq][2 * pp][2] * inv, O[hq][2 * pp][3] * inv);
                  v[2] = pack_bf16x2(O[hq][2 * pp + 1][0] * inv, O[hq][2 * pp + 1][1] * inv);
                  v[3] = pack_bf16x2(O[hq][2 * pp + 1][2] * inv, O[hq][2 * pp + 1][3] * inv);
                  *reinterpret_cast<u32x4*>(orow + 32 * pp) = v;
                }
              } else {
                __bf16* orow = p.out + (int64_t)b * p.out_stride_b + (int64_t)h * p.out_stride_h + 128 * role + 4 * g;
#pragma unroll
                for (int db = 0; db < 8; ++db) {
                  u32x2 v;
                  v[0] = pack_bf16x2(O[hq][db][0] * inv, O[hq][db][1] * inv);
                  v[1] = pack_bf16x2(O[hq][db][2] * inv, O[hq][db][3] * inv);
                  *reinterpret_cast<u32x2*>(orow + 16 * db) = v;
                }
              }
            }
            ops += to_ws ? 16 : 32;
            // the LSE of head block `role`
            const int h = 16 * role + c;
            const float l = s_l[0][h] + s_l[1][h];
            const float lse_nat = l > 0.f ? (s_mref[h] + log2f(l)) * 0.69314718055994531f : -INFINITY;
            if (!to_ws) {
              if (p.lse != nullptr) {
                if (g == 0) p.lse[(int64_t)b * p.lse_stride_b + h] = lse_nat;
                ops += 1;
              }
            } else {
              if (g == 0) p.ws_lse[(int64_t)slot * p.heads + h] = lse_nat;
              ops += 1;
            }
          }
#pragma unroll
          for (int hq = 0; hq < 4; ++hq)
#pragma unroll
            for (int db = 0; db < 8; ++db) O[hq][db] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }

      if (nparts > 0 && kLate && iss_valid) {  // this step's DMA after the work
        issue(iss, n_issued++);
        iss_valid = advance(iss);
      }
      if constexpr (kSmall && kScore) if (role == 0) la_step();  // tile j + 3's offsets, tile j + 4 in flight
      // ---- advance: tile j becomes the previous tile
      prev_kv = cur_kv;
      prev_end = cur_end;
      prev_r = cs.r;
      if (cur_kv) {
        ++comp_kv;
        first_kv = cur_end;  // the next KV tile starts a piece
      }
      if (s_valid) s_valid = advance(cs);
      ++j;
      if (!s_valid && !prev_kv) break;
    }
    };
    if (scorer) run(std::true_type{});
    else run(std::false_type{});
    return true;
  };

  if constexpr (kLoop) {
    for (int w = blockIdx.x; w < p.num_ctas; w += gridDim.x) {
      if (w != (int)blockIdx.x) {  // the previous range's waves are done with the LDS tables and ring
        wait_vmcnt<0>();
        __syncthreads();
      }
      if (!range(w)) break;
    }
  } else {
    range(blockIdx.x);
  }
}

}  // namespace

bool decode_ws_takes(const DecodeParams& p) {
  if (p.heads != 64) return false;
  if (p.log2_ps >= 5) return true;
  // pages under 32 tokens: every row offset from the pool base must fit in 32 bits
  return ((int64_t)p.num_pages << p.log2_ps) * p.kv_row_stride * 2 <= (int64_t)UINT32_MAX;
}

template <bool kSmall>
static void launch_ws(const DecodeParams& p, hipStream_t stream) {
  const int cus = current_device_cus();
  if (p.num_ctas <= cus)
    hipLaunchKernelGGL((mla_decode_ws_kernel<kSmall, false>), dim3(p.num_ctas), dim3(kWWaves * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((mla_decode_ws_kernel<kSmall, true>), dim3(cus), dim3(kWWaves * 64), 0, stream, p);
}

hipError_t launch_decode_ws(const DecodeParams& p, hipStream_t stream) {
  if (p.log2_ps >= 5) launch_ws<false>(p, stream);
  else launch_ws<true>(p, stream);
  return hipGetLastError();
}

}  // namespace mla
