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
