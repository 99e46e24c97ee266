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

    def randn(shape, gen_seed):
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

    q = randn((T, heads, QK_DIM), seed + 1)
    k = randn((num_pages, page_size, heads, QK_DIM), seed + 2)
    v = randn((num_pages, page_size, heads, V_DIM), seed + 3)
    cu = [0]
    for E in extends:
        cu.append(cu[-1] + E)
    return PrefillCase(
        q=q, k_pool=k, v_pool=v, page_table=pt.to(dev),
        cu_seqlens_q=torch.tensor(cu, dtype=torch.int32, device=dev),
        seq_lens_k=torch.tensor(lens, dtype=torch.int32, device=dev),
        extends=extends, prefixes=prefixes, page_size=page_size,
    )
