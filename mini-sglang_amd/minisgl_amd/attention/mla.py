"""MI355X MLA attention backend (absorbed decode + chunked prefill).

Implements the five methods of ``BaseAttnBackend``
(python/minisgl/attention/base.py:18-34) following the FlashAttention
backend's metadata and capture flow (python/minisgl/attention/fa.py:36-136),
with the attention math in libmla_amd.so:

* ``prepare_metadata`` builds, from ``batch.padded_reqs``, the per-request
  lengths (fa.py:71-90), the page table (fa.py:92-97, by a bit-exact HIP
  gather kernel) and -- for decode -- a split-KV plan computed on the host by
  the library's planner (the role FlashInfer's plan() plays in fi.py:123-166).
  Host arrays go to the device with pinned non-blocking copies (fa.py:76-90).
* ``forward`` stores the new rows into the pool (fa.py:53) and runs, for a
  decode batch, the absorbed decode kernel: ``q [B, H, 576]`` -> ``o [B, H,
  512]`` (latent space; the caller applies W_UV); for a prefill batch, the
  chunked prefill kernel over the per-head K/V pages: ``q [T, H, 192]`` -> ``o
  [T, H, 128]``.
* the capture hooks point the metadata at static buffers sized for the
  largest captured batch (fa.py:107-136); replay copies the live metadata in.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Tuple

import numpy as np
import torch

from ..config import MLAConfig
from ..core import Batch, get_global_ctx
from ..kernel import lib
from ..kvcache.mla_pool import MLAKVCache
from .base import BaseAttnBackend, BaseAttnMetadata
from .utils import BaseCaptureData

_CPU_I32 = {"device": "cpu", "dtype": torch.int32, "pin_memory": True}


# the prefill kernel reads keys in 64-token tiles that must lie inside one page
PREFILL_PAGE = 64


@dataclass
class MLACaptureData(BaseCaptureData):
    plan: torch.Tensor  # int32 [num_ctas * 4 + max_bs * 3]


@dataclass
class MLAMetadata(BaseAttnMetadata):
    cu_seqlens_k: torch.Tensor
    cu_seqlens_q: torch.Tensor
    cache_seqlens: torch.Tensor  # int32 [bs] device_len per request
    max_seqlen_k: int
    max_seqlen_q: int
    page_table: torch.Tensor  # int32 [bs, ceil(max_seqlen_k / ps)] page ids
    is_decode: bool
    plan: torch.Tensor | None = None  # decode split-KV plan (device)
    num_slots: int = 0
    seqlens_k: List[int] | None = None  # host copy of cache_seqlens (prefill batches)
    num_ctas: int = 0  # grid of the decode launch (the plan's CTA count)
    workspace: Tuple[torch.Tensor, torch.Tensor] | None = None  # split-KV partials (decode)

    def get_last_indices(self, bs: int) -> torch.Tensor:
        return self.cu_seqlens_q[1 : 1 + bs] - 1


class MLAAttnBackend(BaseAttnBackend):
    def __init__(self, config: MLAConfig, num_ctas: int | None = None):
        ctx = get_global_ctx()
        assert isinstance(ctx.kv_cache, MLAKVCache), "the MLA backend needs an MLAKVCache pool"
        self.config = config
        self.kvcache: MLAKVCache = ctx.kv_cache
        self.page_size = ctx.page_size
        self.device = self.kvcache.device
        self.scale = config.softmax_scale
        self.num_heads = config.num_heads
        if num_ctas is None:  # one persistent decode CTA per compute unit
            dev_index = self.device.index if self.device.index is not None else torch.cuda.current_device()
            num_ctas = lib.device_cu_count(dev_index)
        self.num_ctas = num_ctas
        # every batch's tokens live in the pool, which bounds the grid a decode plan can need
        self.pool_tokens = self.kvcache.num_pages * self.page_size
        self.capture: MLACaptureData | None = None
        self.capture_bs: List[int] = []
        self.max_graph_bs = 0
        self.capture_ctas = self.num_ctas
        # split-KV workspaces: eager batches use (and grow) their own; captured graphs keep theirs
        # fixed from init_capture_graph, so an eager batch never resizes memory a graph points at
        self.ws_eager: Tuple[torch.Tensor, torch.Tensor] | None = None
        self.ws_graph: Tuple[torch.Tensor, torch.Tensor] | None = None
        self.last_lse: torch.Tensor | None = None  # natural-log LSE of the last forward

    # ------------------------------------------------------------------ workspace
    def _new_workspace(self, slots: int) -> Tuple[torch.Tensor, torch.Tensor]:
        capturing = torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
        assert not capturing, "decode workspaces are allocated outside capture"
        ws_o = torch.empty((slots, self.num_heads, self.config.kv_lora_rank), dtype=torch.float32, device=self.device)
        ws_lse = torch.empty((slots, self.num_heads), dtype=torch.float32, device=self.device)
        return ws_o, ws_lse

    def _eager_workspace(self, slots: int) -> Tuple[torch.Tensor, torch.Tensor]:
        if self.ws_eager is None or self.ws_eager[0].shape[0] < slots:
            self.ws_eager = self._new_workspace(max(slots, 2 * self.num_ctas))
        return self.ws_eager

    # ------------------------------------------------------------------ forward
    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer_id: int, batch: Batch) -> torch.Tensor:
        metadata = batch.attn_metadata
        assert isinstance(metadata, MLAMetadata)
        self.kvcache.store_kv(k, v, batch.out_loc, layer_id)
        if not metadata.is_decode:
            return self._forward_prefill(q, layer_id, metadata)
        B, H, _ = q.shape
        out = torch.empty((B, H, self.config.kv_lora_rank), dtype=q.dtype, device=q.device)
        lse = torch.empty((B, H), dtype=torch.float32, device=q.device)
        ws_o, ws_lse = metadata.workspace
        lib.mla_decode(
            q, self.kvcache.latent_cache(layer_id), metadata.page_table, metadata.cache_seqlens, metadata.plan,
            metadata.num_ctas, ws_o, ws_lse, self.scale, out, lse,
        )
        self.last_lse = lse
        return out

    def _forward_prefill(self, q: torch.Tensor, layer_id: int, metadata: MLAMetadata) -> torch.Tensor:
        """Chunked prefill, non-absorbed: ``q [T, H, 192]`` over the per-head K/V pages -> ``[T, H, 128]``.

        The new tokens' K/V were stored above; every request attends its prefix and itself causally
        (bottom-right aligned, ``attention/fa.py:155``)."""
        T, H, _ = q.shape
        out = torch.empty((T, H, self.config.v_head_dim), dtype=q.dtype, device=q.device)
        lse = torch.empty((T, H), dtype=torch.float32, device=q.device)
        k_pages, v_pages = self.kvcache.prefill_k_cache(layer_id), self.kvcache.prefill_v_cache(layer_id)
        page_table = metadata.page_table
        if self.page_size < PREFILL_PAGE:
            k_pages, v_pages, page_table = self._prefill_pages_of(k_pages, v_pages, metadata)
        lib.mla_prefill(
            q, k_pages, v_pages, page_table, metadata.cu_seqlens_q, metadata.cache_seqlens, self.scale, out, lse,
        )
        self.last_lse = lse
        return out

    def _prefill_pages_of(self, k_pool: torch.Tensor, v_pool: torch.Tensor, md: MLAMetadata):
        """Pools with pages smaller than the prefill kernel's 64-token key tile (the reference's
        default page size is 1, python/minisgl/engine/config.py:25): every request's K/V rows are
        gathered on the device into consecutive 64-token pages of a scratch pool, with a page table
        over it, and the prefill kernel runs on those."""
        ps, H = self.page_size, k_pool.shape[-2]
        lens = md.seqlens_k
        pages = [-(-L // PREFILL_PAGE) for L in lens]
        first = [0]
        for n in pages:
            first.append(first[-1] + n)
        dev = k_pool.device
        k_tmp = torch.empty((max(first[-1], 1), PREFILL_PAGE, H, k_pool.shape[-1]), dtype=k_pool.dtype, device=dev)
        v_tmp = torch.empty((max(first[-1], 1), PREFILL_PAGE, H, v_pool.shape[-1]), dtype=v_pool.dtype, device=dev)
        kf, vf = k_pool.view(-1, H * k_pool.shape[-1]), v_pool.view(-1, H * v_pool.shape[-1])
        ktf, vtf = k_tmp.view(-1, H * k_pool.shape[-1]), v_tmp.view(-1, H * v_pool.shape[-1])
        for b, L in enumerate(lens):
            if L == 0:
                continue
            t = torch.arange(L, device=dev)
            src = md.page_table[b, t // ps].long() * ps + t % ps  # the request's pool rows
            dst0 = first[b] * PREFILL_PAGE
            lib.gather_rows(ktf[dst0 : dst0 + L], kf, src)
            lib.gather_rows(vtf[dst0 : dst0 + L], vf, src)
        width = max(max(pages), 1)
        pt = torch.tensor([[first[b] + min(j, max(n - 1, 0)) for j in range(width)] for b, n in enumerate(pages)],
                          dtype=torch.int32).to(dev, non_blocking=True)
        return k_tmp, v_tmp, pt

    def _plan(self, seqlens_k: List[int], grid: int | None = None):
        """Split plan on the smallest grid of ``num_ctas * 2^k`` CTAs that holds the batch (one CTA per
        compute unit unless a CTA's range would pass the kernels' per-CTA limits of
        ``MAX_CTA_BLOCKS`` blocks or ``MAX_CTA_REQUESTS`` requests; further CTAs run as further
        rounds). With ``grid`` the plan is laid out for a launch of ``grid`` CTAs: the CTAs past the
        planned ones get empty ranges. Returns ``(plan, slots, launch CTAs)``."""
        ctas = self.num_ctas
        limit = grid if grid is not None else max(self.num_ctas, self._grid_bound(sum(seqlens_k), len(seqlens_k)))
        while True:
            try:
                plan_np, slots = lib.decode_plan(seqlens_k, self.page_size, ctas)
                break
            except lib.MLAKernelError as e:
                if "cannot hold" not in str(e) or ctas >= limit:
                    raise
                ctas *= 2
        assert slots <= 2 * ctas, "a CTA holds at most two pieces of split requests"
        if grid is None or grid == ctas:
            return plan_np, slots, ctas
        return pad_plan(plan_np, ctas, grid, len(seqlens_k)), slots, grid

    def _grid_bound(self, tokens: int, reqs: int) -> int:
        """Smallest ``num_ctas * 2^k`` grid that holds any batch of ``reqs`` requests and ``tokens``
        tokens in all: the planner closes a CTA only at ``MAX_CTA_BLOCKS`` blocks or
        ``MAX_CTA_REQUESTS`` requests (pieces have no length limit), and each request rounds up by
        less than one block."""
        blocks = -(-tokens // lib.PLAN_BLOCK) + reqs
        need = -(-blocks // lib.MAX_CTA_BLOCKS) + -(-reqs // (lib.MAX_CTA_REQUESTS - 1)) + 1
        grid = self.num_ctas
        while grid < need:
            grid *= 2
        return grid

    # ------------------------------------------------------------------ metadata
    def prepare_metadata(self, batch: Batch) -> None:
        reqs = batch.padded_reqs
        padded_size = len(reqs)
        seqlens_q = [r.extend_len for r in reqs]
        seqlens_k = [r.device_len for r in reqs]
        cached_lens = [r.cached_len for r in reqs]
        max_seqlen_k = max(seqlens_k)
        max_seqlen_q = max(seqlens_q)
        device = self.device

        cache_seqlens = torch.tensor(seqlens_k, **_CPU_I32).to(device, non_blocking=True)
        cu_seqlens_k = torch.tensor([0] + seqlens_k, **_CPU_I32).cumsum_(dim=0).to(device, non_blocking=True)
        if max_seqlen_q == 1:
            cu_seqlens_q = torch.arange(0, padded_size + 1, device=device, dtype=torch.int32)
        elif all(c == 0 for c in cached_lens):  # prefill with no cache hit
            cu_seqlens_q = cu_seqlens_k
        else:
            cu_seqlens_q = torch.tensor([0] + seqlens_q, **_CPU_I32).cumsum_(dim=0).to(device, non_blocking=True)

        table_idx = torch.tensor([r.table_idx for r in reqs], **_CPU_I32).to(device, non_blocking=True)
        page_table = lib.page_table_from_tokens(get_global_ctx().page_table, table_idx, max_seqlen_k, self.page_size)

        is_decode = batch.is_decode
        plan_dev, slots, ctas = None, 0, 0
        workspace = None
        if is_decode:
            assert max_seqlen_q == 1, "decode batches extend every request by one token"
            graphed = self.capture is not None and padded_size in self.capture_bs
            if graphed:  # replayed: planned for the captured grid and workspace
                plan_np, slots, ctas = self._plan(seqlens_k, self.capture_ctas)
                workspace = self.ws_graph
            else:
                plan_np, slots, ctas = self._plan(seqlens_k)
                workspace = self._eager_workspace(slots)
            assert slots <= workspace[0].shape[0]
            plan_dev = torch.from_numpy(plan_np).pin_memory().to(device, non_blocking=True)
        batch.attn_metadata = MLAMetadata(
            cu_seqlens_k=cu_seqlens_k,
            cu_seqlens_q=cu_seqlens_q,
            cache_seqlens=cache_seqlens,
            max_seqlen_k=max_seqlen_k,
            max_seqlen_q=max_seqlen_q,
            page_table=page_table,
            is_decode=is_decode,
            plan=plan_dev,
            num_slots=slots,
            seqlens_k=None if is_decode else seqlens_k,
            num_ctas=ctas if is_decode else 0,
            workspace=workspace,
        )

    # ------------------------------------------------------------------ graph capture
    def init_capture_graph(self, max_seq_len: int, bs_list: List[int]) -> None:
        assert self.capture is None, "Capture already initialized."
        max_bs = max(bs_list)
        cols = -(-max_seq_len // self.page_size)
        # the captured launch has a fixed grid: the one the largest batch the graphs can replay needs,
        # whose tokens are bounded by both the pool and max_bs * max_seq_len
        self.capture_ctas = self._grid_bound(min(self.pool_tokens, max_bs * max_seq_len), max_bs)
        plan = torch.zeros((self.capture_ctas * lib.PLAN_CTA_INTS + max_bs * lib.PLAN_REQ_INTS,), dtype=torch.int32,
                           device=self.device)
        self.ws_graph = self._new_workspace(2 * self.capture_ctas)  # a plan needs at most 2 slots per CTA
        self.capture = MLACaptureData.create(max_bs, cols, self.device, plan=plan)
        self.max_graph_bs = max_bs
        self.capture_bs = sorted(bs_list)

    def prepare_for_capture(self, batch: Batch) -> None:
        assert (bs := batch.size) in self.capture_bs and self.capture is not None
        cap = self.capture
        plan_np, _, _ = self._plan([r.device_len for r in batch.reqs], self.capture_ctas)
        n = plan_np.shape[0]
        cap.plan[:n].copy_(torch.from_numpy(plan_np))
        batch.attn_metadata = MLAMetadata(
            cu_seqlens_k=cap.cu_seqlens_k[: bs + 1],
            cu_seqlens_q=cap.cu_seqlens_q[: bs + 1],
            cache_seqlens=cap.seq_lens[:bs],
            max_seqlen_k=cap.page_table.size(1) * self.page_size,
            max_seqlen_q=1,
            page_table=cap.page_table[:bs, :],
            is_decode=True,
            plan=cap.plan,
            num_slots=self.ws_graph[0].shape[0],
            num_ctas=self.capture_ctas,
            workspace=self.ws_graph,
        )

    def prepare_for_replay(self, batch: Batch) -> None:
        metadata, bs = batch.attn_metadata, batch.padded_size
        assert isinstance(metadata, MLAMetadata) and metadata.is_decode
        assert self.capture is not None and bs in self.capture_bs
        cap = self.capture
        table_len = metadata.page_table.size(1)
        cap.cu_seqlens_k[: bs + 1].copy_(metadata.cu_seqlens_k)
        cap.seq_lens[:bs].copy_(metadata.cache_seqlens)
        cap.page_table[:bs, :table_len].copy_(metadata.page_table)
        assert metadata.num_ctas == self.capture_ctas, "replayed batches are planned for the captured grid"
        cap.plan[: metadata.plan.numel()].copy_(metadata.plan)


def pad_plan(plan: np.ndarray, ctas: int, grid: int, batch: int) -> np.ndarray:
    """A plan made for ``ctas`` CTAs laid out for a launch of ``grid >= ctas`` CTAs: the extra CTAs
    get the empty range ``(batch, 0, batch, 0)``; the request info is unchanged."""
    assert grid >= ctas
    out = np.empty(grid * lib.PLAN_CTA_INTS + batch * lib.PLAN_REQ_INTS, dtype=np.int32)
    n = ctas * lib.PLAN_CTA_INTS
    out[:n] = plan[:n]
    out[n : grid * lib.PLAN_CTA_INTS] = np.tile(np.array([batch, 0, batch, 0], dtype=np.int32), grid - ctas)
    out[grid * lib.PLAN_CTA_INTS :] = plan[n:]
    return out


def plan_pieces(plan: np.ndarray, num_ctas: int, seq_lens) -> List[tuple]:
    """Decode a host plan into ``(cta, request, t0, t1)`` pieces (for tests and tools)."""
    B = len(seq_lens)
    cta = plan[: num_ctas * lib.PLAN_CTA_INTS].reshape(num_ctas, 4)
    out = []
    for w in range(num_ctas):
        rb, kb, re, ke = (int(x) for x in cta[w])
        for b in range(rb, min(re, B - 1) + 1):
            L = int(seq_lens[b])
            t0 = kb * lib.PLAN_BLOCK if b == rb else 0
            t1 = min(ke * lib.PLAN_BLOCK, L) if b == re else L
            if t1 > t0:
                out.append((w, b, t0, t1))
    return out
