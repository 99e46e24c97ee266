// Chunked MLA prefill (non-absorbed form), causal and bottom-right aligned over
// a paged prefix: query i of a request with prefix P attends keys j <= P + i.
// Per head: q [192] (128 nope + 64 rope), K [192], V [128].
//
// One CTA per (request, 256 query rows, head); 4 waves x 64 query rows.
//  * K/V tiles of 64 tokens (K 24 KB + V 16 KB) are staged by 16-byte DMA
//    loads into a 3-stage LDS ring. K rows (384 B) are stored with the 16-byte
//    chunk index XOR (token & 7) inside each 8-chunk group, V rows (256 B) with
//    XOR 2 * (token & 3): both the K operand reads and the transposing V reads
//    are then bank-conflict free.
//  * S^T[32 keys x 32 queries] = K . Q^T on 32x32x16 bf16 MFMA, two key halves
//    x two 32-row query sub-blocks per tile; each K read feeds both
//    sub-blocks. The wave's queries live in accumulation registers as the B
//    operand. Each lane holds 16 keys of one query per key half: the row max
//    needs one cross-half shuffle and the softmax numerators P^T are already
//    in the B-operand layout of O^T[128 dims x 32 queries] += V^T . P^T (k
//    order permuted consistently in the V^T reads); each V^T read feeds both
//    sub-blocks.
//  * Online softmax in the log2 domain with lazy rescaling: the running max
//    moves (and O, l are rescaled) only when a tile's max exceeds it by 8.
//  * The heads of one (request, query block) are consecutive CTAs, so the
//    query blocks of one head are 'heads' CTAs apart and, with heads a
//    multiple of 8, land on the same XCD and share its L2 for K/V.
#include "mla_common.h"
#include "mla_device.h"

namespace mla {
namespace {

typedef float f32x16_t __attribute__((__vector_size__(64)));

constexpr int kPWaves = 4;
constexpr int kPRowsPerWave = kPrefillRows / kPWaves;  // 64
constexpr int kPTile = 64;                              // keys per tile (one page: page_size >= 64)
constexpr int kPKRowBytes = kPrefillQkDim * 2;          // 384
constexpr int kPVRowBytes = kPrefillVDim * 2;           // 256
constexpr int kPKBytes = kPTile * kPKRowBytes;          // 24576
constexpr int kPVBytes = kPTile * kPVRowBytes;          // 16384
constexpr int kPStageBytes = kPKBytes + kPVBytes;       // 40960
constexpr int kPStages = 3;
constexpr int kPKDma = kPKBytes / 1024 / kPWaves;  // 6 wave-wide DMA loads per wave
constexpr int kPVDma = kPVBytes / 1024 / kPWaves;  // 4
constexpr int kPDma = kPKDma + kPVDma;             // 10
constexpr float kPRescaleLog2 = 8.0f;
constexpr int kPMaxPages = 4096;  // page ids of a CTA's keys staged in LDS (else read per tile)

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ int kswz(int c, int t) { return (c & ~7) | ((c & 7) ^ (t & 7)); }
__device__ __forceinline__ int vswz(int c, int t) { return c ^ (2 * (t & 3)); }

// S^T += K . Q^T with the query operand read straight from accumulation registers (where the queries
// live for the whole kernel), so the compiler does not copy them per MFMA. A chain accumulates in
// place; its first k-step starts from zero.
__device__ __forceinline__ void mfma_qk_first(f32x16_t& d, const bf16x8& k, const bf16x8& q) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(k), "a"(q));
}
__device__ __forceinline__ void mfma_qk(f32x16_t& d, const bf16x8& k, const bf16x8& q) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "a"(q));
}
// The scores written by the chains above are read by vector ALU instructions next: wait states
// between the last MFMA's write and the first read (24 >= what a 16-pass MFMA needs).
__device__ __forceinline__ void mfma_result_wait(f32x16_t& a, f32x16_t& b, f32x16_t& c, f32x16_t& d) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}

__global__ __launch_bounds__(256, 1) void mla_prefill_kernel(const PrefillParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kPStages * kPStageBytes];
  __shared__ int s_pg[kPMaxPages];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = p.heads;

  // ---- work item: request b, query block qb, head h (heads fastest); the last items (the
  // latest query blocks, which see the most keys) are dispatched first
  auto items_of = [&](int r) {
    return r < p.batch ? ((p.cu_seqlens_q[r + 1] - p.cu_seqlens_q[r] + kPrefillRows - 1) / kPrefillRows) * H : 0;
  };
  int total = 0;
  for (int c0 = 0; c0 < p.batch; c0 += 64) total += wave_sum(items_of(c0 + lane));
  total = __builtin_amdgcn_readfirstlane(total);
  const int item = total - 1 - (int)blockIdx.x;
  int b = -1, local = 0;
  if (item >= 0) {
    int acc = 0;
    for (int c0 = 0; c0 < p.batch && b < 0; c0 += 64) {
      const int r = c0 + lane;
      const int n = items_of(r);
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
      }
      acc += __shfl(incl, 63);
    }
  }
  b = __builtin_amdgcn_readfirstlane(b);
  if (b < 0) return;  // uniform: beyond the last item
  local = __builtin_amdgcn_readfirstlane(local);
  const int h = local % H;
  const int qb = local / H;
  const int q0 = p.cu_seqlens_q[b];
  const int E = p.cu_seqlens_q[b + 1] - q0;
  const int L = p.seq_lens_k[b];
  const int P = L - E;  // prefix length
  const int row0 = qb * kPrefillRows + wave * kPRowsPerWave;  // this wave's first query row in the request
  const int cta_rows_end = min(E, (qb + 1) * kPrefillRows);
  const int nkeys = P + cta_rows_end;  // keys the CTA needs
  const int ntiles = (nkeys + kPTile - 1) / kPTile;
  const int wave_rows = max(0, min(E - row0, kPRowsPerWave));
  const int wave_tiles = wave_rows > 0 ? (P + row0 + wave_rows + kPTile - 1) / kPTile : 0;

  const int g32 = lane >> 5;  // half of the wave
  const int c32 = lane & 31;
  const int ps_mask = (1 << p.log2_ps) - 1;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(MLA_LDS char*)smem;
  const char* kbase = reinterpret_cast<const char*>(p.k) + (int64_t)h * kPKRowBytes;
  const char* vbase = reinterpret_cast<const char*>(p.v) + (int64_t)h * kPVRowBytes;
  const int krow_bytes = (int)(p.k_row_stride * 2), vrow_bytes = (int)(p.v_row_stride * 2);

  // ---- page ids of the CTA's keys
  const int npages = (nkeys + ps_mask) >> p.log2_ps;
  const bool staged = npages <= kPMaxPages;
  if (staged) {
    for (int i = threadIdx.x; i < npages; i += 256)
      s_pg[i] = min(max(p.page_table[(int64_t)b * p.pt_stride + i], 0), p.num_pages - 1);
    __syncthreads();
  }

  // ---- DMA of key tile n (64 tokens of one page); rows past the last key load the last key.
  // LDS position s (16 bytes each) of the K tile holds token s / 24, chunk kswz(s % 24); of the V tile
  // token s / 16, chunk vswz(s % 16).
  uint32_t koff[kPKDma], voff[kPVDma];
#pragma unroll
  for (int k = 0; k < kPKDma; ++k) {
    const int s = (wave + k * kPWaves) * 64 + lane, t = s / 24;
    koff[k] = (uint32_t)(t * krow_bytes + kswz(s - 24 * t, t) * 16);
  }
#pragma unroll
  for (int k = 0; k < kPVDma; ++k) {
    const int s = (wave + k * kPWaves) * 64 + lane, t = s >> 4;
    voff[k] = (uint32_t)(t * vrow_bytes + vswz(s & 15, t) * 16);
  }
  auto issue = [&](int n) {
    const int t0 = n * kPTile;
    const int pid = staged ? __builtin_amdgcn_readfirstlane(s_pg[t0 >> p.log2_ps])
                           : min(max(sload_i32(p.page_table + (int64_t)b * p.pt_stride + (t0 >> p.log2_ps)), 0),
                                 p.num_pages - 1);
    const int64_t row_base = (int64_t)pid * (ps_mask + 1) + (t0 & ps_mask);
    const char* ksrc = kbase + row_base * krow_bytes;
    const char* vsrc = vbase + row_base * vrow_bytes;
    const uint32_t st = lds0 + (n % kPStages) * kPStageBytes;
    const int tlim = L - 1 - t0;
    if (tlim >= kPTile - 1) {
#pragma unroll
      for (int k = 0; k < kPKDma; ++k) dma16_saddr(ksrc, koff[k], st + (wave + k * kPWaves) * 1024);
#pragma unroll
      for (int k = 0; k < kPVDma; ++k) dma16_saddr(vsrc, voff[k], st + kPKBytes + (wave + k * kPWaves) * 1024);
    } else {
#pragma unroll
      for (int k = 0; k < kPKDma; ++k) {
        const int s = (wave + k * kPWaves) * 64 + lane, t = s / 24;
        const uint32_t o = (uint32_t)(min(t, tlim) * krow_bytes + kswz(s - 24 * t, t) * 16);
        dma16_saddr(ksrc, o, st + (wave + k * kPWaves) * 1024);
      }
#pragma unroll
      for (int k = 0; k < kPVDma; ++k) {
        const int s = (wave + k * kPWaves) * 64 + lane, t = s >> 4;
        const uint32_t o = (uint32_t)(min(t, tlim) * vrow_bytes + vswz(s & 15, t) * 16);
        dma16_saddr(vsrc, o, st + kPKBytes + (wave + k * kPWaves) * 1024);
      }
    }
  };

  // ---- queries: qf[qs][ks] = row row0 + 32qs + c32, dims 16ks + 8g32 .. +8 (zeros past the extend)
  bf16x8 qf[2][12];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    const int row = row0 + 32 * qs + c32;
    const bool ok = row < E;
    const __bf16* qrow = p.q + (int64_t)(q0 + (ok ? row : 0)) * p.q_stride_t + (int64_t)h * p.q_stride_h + 8 * g32;
#pragma unroll
    for (int ks = 0; ks < 12; ++ks) qf[qs][ks] = ok ? *reinterpret_cast<const bf16x8*>(qrow + 16 * ks) : bf16x8{};
  }
  // the queries stay in accumulation registers for the whole kernel (the score MFMAs read them there)
#pragma unroll
  for (int qs = 0; qs < 2; ++qs)
#pragma unroll
    for (int ks = 0; ks < 12; ++ks) asm volatile("" : "=a"(qf[qs][ks]) : "0"(qf[qs][ks]));

  int n_issued = 0;
  for (; n_issued < kPStages - 1 && n_issued < ntiles; ++n_issued) issue(n_issued);

  // ---- per-lane LDS read offsets
  // K operand of k-step ks = 4m + r, key half kh: chunk 8m + 2r + g32 of key 32kh + c32 at k_off[r] + 128m
  int k_off[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) k_off[r] = c32 * kPKRowBytes + kswz(2 * r + g32, c32) * 16;
  // V^T operand: 16-lane group gq = lane / 16 covers dims 16(gq & 1) .. +16 of a 32-dim block and the
  // key half vh = gq >> 1; lane a16 reads token 4vh + (a16 >> 2) (+ 16 ksp + 8 second + 32 kh), dims
  // 4(a16 & 3) .. +4; chunk 4db + y (y < 4) is stored at (4db + y) ^ 2vt
  const int gq = lane >> 4, a16 = lane & 15, vh = gq >> 1, vt = a16 >> 2;
  int v_off[2];
  {
    const int y = 2 * (gq & 1) + ((a16 & 3) >> 1);
    const int z = y ^ (2 * vt);
#pragma unroll
    for (int d = 0; d < 2; ++d) v_off[d] = (4 * vh + vt) * kPVRowBytes + ((4 * d) ^ z) * 16 + (a16 & 1) * 8;
  }

  f32x16_t O[4][2];
#pragma unroll
  for (int db = 0; db < 4; ++db) O[db][0] = O[db][1] = f32x16_t{};
  float m_ref[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};

  for (int n = 0; n < ntiles; ++n) {
    wait_vmcnt_dyn(kPDma * (n_issued - 1 - n));
    barrier_lds();
    if (n_issued < ntiles) issue(n_issued++);
    if (n >= wave_tiles) continue;  // uniform per wave: its queries need no further keys

    const MLA_LDS char* TK = (const MLA_LDS char*)smem + (n % kPStages) * kPStageBytes;
    const MLA_LDS char* TV = TK + kPKBytes;
    const int kfirst = n * kPTile;

    // ---- S^T = K . Q^T: key halves kh x query sub-blocks qs; read r = 12kh + ks
    f32x16_t sc[2][2];
    {
      auto kread = [&](int r) {
        const int kh = r / 12, ks = r % 12;
        return *reinterpret_cast<const MLA_LDS bf16x8*>(TK + kh * 32 * kPKRowBytes + k_off[ks & 3] + 128 * (ks >> 2));
      };
      bf16x8 kb[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) kb[r] = kread(r);
#pragma unroll
      for (int r = 0; r < 24; ++r) {
        const bf16x8 a = kb[r & 3];
        if (r + 4 < 24) kb[r & 3] = kread(r + 4);
        const int kh = r / 12, ks = r % 12;
        if (ks == 0) {
          mfma_qk_first(sc[kh][0], a, qf[0][0]);
          mfma_qk_first(sc[kh][1], a, qf[1][0]);
        } else {
          mfma_qk(sc[kh][0], a, qf[0][ks]);
          mfma_qk(sc[kh][1], a, qf[1][ks]);
        }
      }
    }
    mfma_result_wait(sc[0][0], sc[0][1], sc[1][0], sc[1][1]);

    // ---- online softmax; lane holds keys kfirst + 32kh + 8(i/4) + 4*g32 + i%4 (i < 16) of query
    // column c32 of sub-block qs; the scores become numerators in place
    bf16x8 pb[2][2][2];  // [kh][qs][ksp]
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      const int qpos = P + row0 + 32 * qs + c32;                   // this lane's query position
      const bool diag = kfirst + kPTile - 1 > P + row0 + 32 * qs;  // uniform: some key may follow a query
      float m = -INFINITY;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (diag && kfirst + 32 * kh + 8 * (i >> 2) + 4 * g32 + (i & 3) > qpos) sc[kh][qs][i] = -INFINITY;
          m = fmaxf(m, sc[kh][qs][i]);
        }
      const float mblk = fmaxf(m, __shfl_xor(m, 32)) * p.scale_log2;
      const bool up = mblk > m_ref[qs] + kPRescaleLog2;
      if (__ballot(up) != 0) {  // rare after the first tiles: move the reference, rescale O and l
        const float m_new = up ? mblk : m_ref[qs];
        const float f = __builtin_amdgcn_exp2f(m_ref[qs] - m_new);
        l_run[qs] *= f;
#pragma unroll
        for (int db = 0; db < 4; ++db) O[db][qs] *= f;
        m_ref[qs] = m_new;
      }
      const float neg_m = -m_ref[qs];
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          sc[kh][qs][i] = __builtin_amdgcn_exp2f(fmaf(sc[kh][qs][i], p.scale_log2, neg_m));
          l_run[qs] += sc[kh][qs][i];
        }
#pragma unroll
        for (int ksp = 0; ksp < 2; ++ksp) {
          const f32x16_t& e = sc[kh][qs];
          const u32x4 w{pack_bf16x2(e[8 * ksp + 0], e[8 * ksp + 1]), pack_bf16x2(e[8 * ksp + 2], e[8 * ksp + 3]),
                        pack_bf16x2(e[8 * ksp + 4], e[8 * ksp + 5]), pack_bf16x2(e[8 * ksp + 6], e[8 * ksp + 7])};
          pb[kh][qs][ksp] = __builtin_bit_cast(bf16x8, w);
        }
      }
    }

    // ---- O^T[32 dims x 32 queries] += V^T . P^T per 32-dim block db = 2pp + d; k-step (kh, ksp) covers
    // keys 32kh + 16ksp + 4vh + (0..3) and 32kh + 16ksp + 8 + 4vh + (0..3), matching the lanes' P^T values
    auto vread = [&](int db, int kh, int ksp, int second) {
      const int off = v_off[db & 1] + 128 * (db >> 1) + (32 * kh + 16 * ksp + 8 * second) * kPVRowBytes;
      return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MLA_LDS bf16x4*)(TV + off));
    };
    auto vop = [&](int st) {  // st = (db, kh, ksp)
      const int db = st >> 2, kh = (st >> 1) & 1, ksp = st & 1;
      return __builtin_shufflevector(vread(db, kh, ksp, 0), vread(db, kh, ksp, 1), 0, 1, 2, 3, 4, 5, 6, 7);
    };
    bf16x8 vb[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) vb[st] = vop(st);
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const int db = st >> 2, kh = (st >> 1) & 1, ksp = st & 1;
      const bf16x8 a = vb[st & 3];
      if (st + 4 < 16) vb[st & 3] = vop(st + 4);
      O[db][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[kh][0][ksp], O[db][0], 0, 0, 0);
      O[db][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[kh][1][ksp], O[db][1], 0, 0, 0);
    }
  }

  // ---- finalise: lane holds query column c32 and dims 32db + 8(i/4) + 4*g32 + i%4
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    const int row = row0 + 32 * qs + c32;
    const float l_tot = l_run[qs] + __shfl_xor(l_run[qs], 32);
    if (row >= E || wave_rows == 0) continue;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    __bf16* orow = p.out + (int64_t)(q0 + row) * p.out_stride_t + (int64_t)h * p.out_stride_h + 4 * g32;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        u32x2 v;
        v[0] = pack_bf16x2(O[db][qs][4 * i4 + 0] * inv, O[db][qs][4 * i4 + 1] * inv);
        v[1] = pack_bf16x2(O[db][qs][4 * i4 + 2] * inv, O[db][qs][4 * i4 + 3] * inv);
        *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * i4) = v;
      }
    if (p.lse != nullptr && g32 == 0)
      p.lse[(int64_t)(q0 + row) * p.lse_stride_t + h] =
          l_tot > 0.f ? (m_ref[qs] + log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
  }
}

}  // namespace

hipError_t launch_prefill(const PrefillParams& p, int32_t total_q, hipStream_t stream) {
  // upper bound on sum_b ceil(E_b / 256) over the batch, times the heads
  const int64_t items = ((int64_t)(total_q + kPrefillRows - 1) / kPrefillRows + p.batch) * p.heads;
  if (items <= 0) return hipSuccess;
  hipLaunchKernelGGL(mla_prefill_kernel, dim3((unsigned)items), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mla
