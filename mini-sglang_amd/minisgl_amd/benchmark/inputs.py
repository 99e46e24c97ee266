"""Seeded synthetic inputs of the MLA decode / prefill workloads.

Seeds follow one convention everywhere: generator seed 0 draws the sequence
lengths and page tables, seed 1 the queries, seed 2 the KV rows; values are
N(0, 1) rounded to bf16. Page tables are a random permutation of the pool's
pages (non-contiguous), as a long-running server's allocator produces
(python/minisgl/scheduler/cache.py:106-146).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Sequence

import torch

KV_DIM = 576


@dataclass
class DecodeCase:
    q: torch.Tensor  # bf16 [B, H, 576]
    kv_pool: torch.Tensor  # bf16 [num_pages, ps, 576]
    page_table: torch.Tensor  # int32 [B, max_pages]
    seq_lens: torch.Tensor  # int32 [B]
    lens: List[int]
    page_size: int

    @property
    def kv_bytes(self) -> int:
        return sum(self.lens) * KV_DIM * 2

    def algorithmic_bytes(self) -> int:
        """KV rows read once + q + o + lse + page-table entries + seq_lens."""
        B, H, _ = self.q.shape
        pages = sum(-(-L // self.page_size) for L in self.lens)
        return self.kv_bytes + B * H * (576 + 512) * 2 + B * H * 4 + pages * 4 + 4 * B

    def flops(self) -> int:
        H = self.q.shape[1]
        return sum(self.lens) * H * 2 * (576 + 512)


def _lens(batch: int, lo: int, hi: int, gen: torch.Generator) -> List[int]:
    return torch.randint(lo, hi + 1, (batch,), generator=gen).tolist()


def page_table_for(lens: Sequence[int], page_size: int, num_pages: int, gen: torch.Generator) -> torch.Tensor:
    need = [-(-L // page_size) for L in lens]
    assert sum(need) <= num_pages
    perm = torch.randperm(num_pages, generator=gen).to(torch.int32)
    pt = torch.zeros((len(lens), max(1, max(need) if need else 1)), dtype=torch.int32)
    off = 0
    for b, n in enumerate(need):
        pt[b, :n] = perm[off : off + n]
        off += n
    return pt


def make_decode_case(
    batch: int,
    heads: int,
    page_size: int,
    lens: Sequence[int] | None = None,
    len_range: tuple = (1024, 8192),
    extra_pages: int = 1,
    device: str | torch.device = "cpu",
    seed: int = 0,
) -> DecodeCase:
    g_len = torch.Generator().manual_seed(seed)
    lens = list(lens) if lens is not None else _lens(batch, len_range[0], len_range[1], g_len)
    assert len(lens) == batch
    num_pages = sum(-(-L // page_size) for L in lens) + extra_pages
    pt = page_table_for(lens, page_size, num_pages, g_len)
    dev = torch.device(device)
    if dev.type == "cpu":
        q = torch.randn((batch, heads, KV_DIM), generator=torch.Generator().manual_seed(seed + 1)).to(torch.bfloat16)
        kv = torch.randn((num_pages, page_size, KV_DIM), generator=torch.Generator().manual_seed(seed + 2)).to(
            torch.bfloat16
        )
    else:  # draw on the device: the full-size pools are hundreds of MB
        gq = torch.Generator(device=dev).manual_seed(seed + 1)
        gk = torch.Generator(device=dev).manual_seed(seed + 2)
        q = torch.randn((batch, heads, KV_DIM), generator=gq, device=dev, dtype=torch.float32).to(torch.bfloat16)
        kv = torch.empty((num_pages, page_size, KV_DIM), device=dev, dtype=torch.bfloat16)
        step = max(1, (1 << 26) // (page_size * KV_DIM))
        for p0 in range(0, num_pages, step):
            p1 = min(num_pages, p0 + step)
            kv[p0:p1] = torch.randn((p1 - p0, page_size, KV_DIM), generator=gk, device=dev).to(torch.bfloat16)
    return DecodeCase(
        q=q,
        kv_pool=kv,
        page_table=pt.to(dev),
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=dev),
        lens=lens,
        page_size=page_size,
    )


QK_DIM = 192
V_DIM = 128


@dataclass
class PrefillCase:
    q: torch.Tensor  # bf16 [T, H, 192], requests packed by cu_seqlens_q
    k_pool: torch.Tensor  # bf16 [num_pages, ps, H, 192]
    v_pool: torch.Tensor  # bf16 [num_pages, ps, H, 128]
    page_table: torch.Tensor  # int32 [B, max_pages]
    cu_seqlens_q: torch.Tensor  # int32 [B + 1]
    seq_lens_k: torch.Tensor  # int32 [B]: prefix + extend
    extends: List[int]
    prefixes: List[int]
    page_size: int

    def flops(self) -> int:
        """Unmasked (query, key) pairs x H x 2 x (192 + 128)."""
        H = self.q.shape[1]
        pairs = sum(E * P + E * (E + 1) // 2 for E, P in zip(self.extends, self.prefixes))
        return pairs * H * 2 * (QK_DIM + V_DIM)

    def algorithmic_bytes(self) -> int:
        """K/V of every key once, q, o, lse."""
        T, H, _ = self.q.shape
        keys = sum(E + P for E, P in zip(self.extends, self.prefixes))
        return keys * H * (QK_DIM + V_DIM) * 2 + T * H * (QK_DIM + V_DIM) * 2 + T * H * 4


def randn_bf16(shape, gen_seed: int, dev: torch.device) -> torch.Tensor:
    """N(0, 1) rounded to bf16; on a GPU drawn there in chunks of at most 64 Mi values."""
    if dev.type == "cpu":
        return torch.randn(shape, generator=torch.Generator().manual_seed(gen_seed)).to(torch.bfloat16)
    g = torch.Generator(device=dev).manual_seed(gen_seed)
    out = torch.empty(shape, device=dev, dtype=torch.bfloat16)
    flat = out.view(shape[0], -1)
    step = max(1, (1 << 26) // flat.shape[1])
    for r0 in range(0, shape[0], step):
        r1 = min(shape[0], r0 + step)
        flat[r0:r1] = torch.randn((r1 - r0, flat.shape[1]), generator=g, device=dev).to(torch.bfloat16)
    return out


def make_prefill_case(
    heads: int,
    page_size: int,
    extends: Sequence[int],
    prefixes: Sequence[int],
    extra_pages: int = 1,
    device: str | torch.device = "cpu",
    seed: int = 0,
) -> PrefillCase:
    extends, prefixes = list(extends), list(prefixes)
    lens = [E + P for E, P in zip(extends, prefixes)]
    g_len = torch.Generator().manual_seed(seed)
    num_pages = sum(-(-L // page_size) for L in lens) + extra_pages
    pt = page_table_for(lens, page_size, num_pages, g_len)
    dev = torch.device(device)
    T = sum(extends)
    q = randn_bf16((T, heads, QK_DIM), seed + 1, dev)
    k = randn_bf16((num_pages, page_size, heads, QK_DIM), seed + 2, dev)
    v = randn_bf16((num_pages, page_size, heads, V_DIM), seed + 3, dev)
    cu = [0]
    for E in extends:
        cu.append(cu[-1] + E)
    return PrefillCase(
        q=q, k_pool=k, v_pool=v, page_table=pt.to(dev),
        cu_seqlens_q=torch.tensor(cu, dtype=torch.int32, device=dev),
        seq_lens_k=torch.tensor(lens, dtype=torch.int32, device=dev),
        extends=extends, prefixes=prefixes, page_size=page_size,
    )


@dataclass
class MixedCase:
    """A ragged batch whose requests share radix-prefix pages.

    ``decode`` holds the decode requests over the latent pool, ``prefill`` the
    prefill chunks over the per-head pools; both sets of page tables index the
    same page ids. Pages ``[0, groups * prefix_pages)`` are the shared prefixes
    (group ``g`` owns a contiguous run of ids, permuted inside the run), then
    the prefill chunks' own pages, then the decode requests' own pages; the
    per-head pools only cover the first two ranges, which are the only pages
    a prefill chunk reads.
    """

    decode: DecodeCase
    prefill: PrefillCase
    group_of_decode: List[int]
    group_of_prefill: List[int]
    prefix_len: int


def make_mixed_case(
    n_decode: int,
    n_prefill: int,
    heads: int,
    page_size: int,
    decode_range: tuple,
    chunk: int,
    prefix_len: int,
    groups: int,
    device: str | torch.device = "cpu",
    seed: int = 0,
) -> MixedCase:
    assert prefix_len % page_size == 0, "shared prefixes end on a page boundary"
    gen = torch.Generator().manual_seed(seed)
    dec_lens = _lens(n_decode, decode_range[0], decode_range[1], gen)
    g_dec = [b % groups for b in range(n_decode)]
    g_pre = [(n_decode + i) % groups for i in range(n_prefill)]
    pp = prefix_len // page_size
    shared = [(g * pp + torch.randperm(pp, generator=gen)).to(torch.int32) for g in range(groups)]
    next_id = groups * pp
    chunk_pages = -(-(prefix_len + chunk) // page_size) - pp
    pre_rows = []
    for i in range(n_prefill):
        own = next_id + torch.randperm(chunk_pages, generator=gen).to(torch.int32)
        next_id += chunk_pages
        pre_rows.append(torch.cat([shared[g_pre[i]], own]))
    prefill_pages = next_id
    dec_rows = []
    dec_own = [max(0, -(-L // page_size) - pp) for L in dec_lens]
    perm = prefill_pages + torch.randperm(sum(dec_own), generator=gen).to(torch.int32)
    off = 0
    for b, L in enumerate(dec_lens):
        n_sh = min(pp, -(-L // page_size))
        dec_rows.append(torch.cat([shared[g_dec[b]][:n_sh], perm[off : off + dec_own[b]]]))
        off += dec_own[b]
    num_pages = prefill_pages + sum(dec_own) + 1
    dev = torch.device(device)

    def table(rows):
        w = max(1, max(r.numel() for r in rows))
        pt = torch.zeros((len(rows), w), dtype=torch.int32)
        for b, r in enumerate(rows):
            pt[b, : r.numel()] = r
        return pt.to(dev)

    decode = DecodeCase(
        q=randn_bf16((n_decode, heads, KV_DIM), seed + 1, dev),
        kv_pool=randn_bf16((num_pages, page_size, KV_DIM), seed + 2, dev),
        page_table=table(dec_rows),
        seq_lens=torch.tensor(dec_lens, dtype=torch.int32, device=dev),
        lens=dec_lens,
        page_size=page_size,
    )
    extra = max(1, prefill_pages - n_prefill * (pp + chunk_pages) + 1)
    pre = make_prefill_case(heads, page_size, extends=[chunk] * n_prefill, prefixes=[prefix_len] * n_prefill,
                            extra_pages=extra, device=device, seed=seed + 10)
    assert pre.k_pool.shape[0] >= prefill_pages
    prefill = PrefillCase(q=pre.q, k_pool=pre.k_pool, v_pool=pre.v_pool, page_table=table(pre_rows),
                          cu_seqlens_q=pre.cu_seqlens_q, seq_lens_k=pre.seq_lens_k, extends=pre.extends,
                          prefixes=pre.prefixes, page_size=page_size)
    return MixedCase(decode=decode, prefill=prefill, group_of_decode=g_dec, group_of_prefill=g_pre,
                     prefix_len=prefix_len)
