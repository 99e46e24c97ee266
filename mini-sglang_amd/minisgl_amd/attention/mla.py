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
* ``forward`` stores the new latent rows into the pool (fa.py:53) and runs,
  for a decode batch, the absorbed decode kernel: ``q [B, H, 576]`` -> ``o
  [B, H, 512]`` (latent space; the caller applies W_UV); for a prefill batch,
  the chunked prefill over the keys decompressed from the latent pool: a HIP
  gather of every key's latent row into 64-token scratch pages, one GEMM
  ``[k_nope | v] = c W_kvb^T`` (the layer registers its ``W_kvb``), then the
  prefill kernel: ``q [T, H, 192]`` -> ``o [T, H, 128]``. Any page size.
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


# the prefill kernel reads keys in 64-token tiles that must lie inside one page: the decompression
# scratch is laid out in pages of this many rows
PREFILL_PAGE = 64
# decompression scratch rows (keys of one prefill pass) unless the backend is given another bound;
# at 64 heads a row is (64 * 256 + 64 + 512) * 2 = 33,920 bytes, so 65,536 rows are 2.2 GB
DEFAULT_PREFILL_SCRATCH_ROWS = 65536


def prefill_scratch_bytes(num_heads: int, rows: int) -> int:
    """Device bytes of a decompression scratch of ``rows`` keys: per key one row
    ``[head 0: k_nope 128 | v 128, ..., rope 64]`` plus its 512 latent dims (the GEMM input)."""
    return rows * (num_heads * 256 + 64 + 512) * 2


def decode_workspace_bytes(num_heads: int, slots: int) -> int:
    """Device bytes of a decode workspace of ``slots`` split-KV slots: a bf16 partial row of 512 dims
    and an fp32 LSE per (slot, head)."""
    return slots * num_heads * (512 * 2 + 4)


def plan_grid_bound(num_ctas: int, tokens: int, reqs: int) -> int:
    """Smallest ``num_ctas * 2^k`` plan grid that holds any batch of ``reqs`` requests and ``tokens``
    tokens in all: the planner closes a CTA range only at ``MAX_CTA_BLOCKS`` blocks or
    ``MAX_CTA_REQUESTS`` requests (pieces have no length limit), and each request rounds up by less
    than one block."""
    blocks = -(-tokens // lib.PLAN_BLOCK) + reqs
    need = -(-blocks // lib.MAX_CTA_BLOCKS) + -(-reqs // (lib.MAX_CTA_REQUESTS - 1)) + 1
    grid = num_ctas
    while grid < need:
        grid *= 2
    return grid


def backend_device_bytes(num_heads: int, num_ctas: int, max_running_req: int, max_seq_len: int,
                         prefill_scratch_rows: int = DEFAULT_PREFILL_SCRATCH_ROWS, graph_max_bs: int = 0) -> int:
    """Device memory an ``MLAAttnBackend`` holds beside the KV pool, for an engine to subtract before
    it sizes the pool (``python/minisgl/engine/engine.py:148-165`` sizes the pool from the free
    memory before the backend exists): the prefill decompression scratch, the eager decode
    workspace for the largest plan grid a batch of ``max_running_req`` requests of at most
    ``max_seq_len`` tokens can need, and -- with graphs up to ``graph_max_bs`` requests -- the
    captured graphs' workspace and plan. A plan uses at most 2 slots per CTA range."""
    eager = plan_grid_bound(num_ctas, max_running_req * max_seq_len, max_running_req)
    total = prefill_scratch_bytes(num_heads, prefill_scratch_rows) + decode_workspace_bytes(num_heads, 2 * eager)
    if graph_max_bs > 0:
        graph = plan_grid_bound(num_ctas, graph_max_bs * max_seq_len, graph_max_bs)
        total += decode_workspace_bytes(num_heads, 2 * graph)
        total += 4 * (graph * lib.PLAN_CTA_INTS + graph_max_bs * lib.PLAN_REQ_INTS)
    return total


def prefill_passes(seqlens_k: List[int], cap_rows: int) -> List[Tuple[int, int, List[int]]]:
    """Split a prefill batch into passes of consecutive whole requests whose keys fit ``cap_rows``
    scratch rows (each request rounded up to 64-row pages); a request longer than the scratch is a
    pass of its own (the scratch then grows to hold it). Returns ``(r0, r1, seg_first)`` per pass:
    requests ``r0 .. r1 - 1``, request ``r0 + i`` starting at scratch page ``seg_first[i]``."""
    passes: List[Tuple[int, int, List[int]]] = []
    r0, first = 0, []
    used = 0
    for r, L in enumerate(seqlens_k):
        pages = -(-L // PREFILL_PAGE)
        if first and (used + pages) * PREFILL_PAGE > cap_rows:
            passes.append((r0, r, first))
            r0, first, used = r, [], 0
        first.append(used)
        used += pages
    if first:
        passes.append((r0, len(seqlens_k), first))
    return passes


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
    num_ctas: int = 0  # grid of the decode launch (the plan's CTA count)
    workspace: Tuple[torch.Tensor, torch.Tensor] | None = None  # split-KV partials (decode)
    # prefill: passes (r0, r1, scratch rows, max pages per request, offset of the pass's seg_first in
    # prefill_seg_first, query rows)
    prefill_plan: List[Tuple[int, int, int, int, int, int]] | None = None
    prefill_seg_first: torch.Tensor | None = None  # int32 (device): each pass's first scratch pages
    prefill_seg_pt: torch.Tensor | None = None  # int32 [bs, max pages] scratch page table (device)

    def get_last_indices(self, bs: int) -> torch.Tensor:
        return self.cu_seqlens_q[1 : 1 + bs] - 1


class MLAAttnBackend(BaseAttnBackend):
    def __init__(self, config: MLAConfig, num_ctas: int | None = None,
                 prefill_scratch_rows: int = DEFAULT_PREFILL_SCRATCH_ROWS, reserve_scratch: bool = False):
        """``reserve_scratch`` allocates the prefill decompression scratch (``prefill_scratch_rows``
        keys) and the eager decode workspace here, as the reference's FlashInfer backend allocates
        its workspace in its constructor (``attention/fi.py:90-92``); otherwise they are allocated at
        the first batch that needs them. ``backend_device_bytes`` gives their size beforehand."""
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
        self.capture: MLACaptureData | None = None
        self.capture_bs: List[int] = []
        self.max_graph_bs = 0
        self.capture_ctas = self.num_ctas
        # split-KV workspaces: eager batches use (and grow) their own; captured graphs keep theirs
        # fixed from init_capture_graph, so an eager batch never resizes memory a graph points at
        self.ws_eager: Tuple[torch.Tensor, torch.Tensor] | None = None
        self.ws_graph: Tuple[torch.Tensor, torch.Tensor] | None = None
        # the eager workspace's last use: an event recorded on the stream of the decode that used it.
        # prepare_metadata of the next batch can run on another stream while that decode still writes
        # partials (python/minisgl/scheduler/scheduler.py:98-103); a workspace replaced by a larger one
        # is kept (retired) until its event has completed, so its memory is not handed out meanwhile
        self.ws_eager_fence = None
        self.ws_retired: List[tuple] = []
        self.last_lse: torch.Tensor | None = None  # natural-log LSE of the last forward
        # prefill decompression: the layers' W_kvb [H * (128 + 128), 512] and a scratch of
        # prefill_scratch_rows keys (allocated at the first prefill, grown for a longer request)
        assert prefill_scratch_rows >= PREFILL_PAGE
        self.prefill_scratch_rows = prefill_scratch_rows
        self.kv_b: dict = {}
        self.scratch_rows: torch.Tensor | None = None  # [rows, H * 256 + 64]: [k_nope | v] per head, rope
        self.scratch_c: torch.Tensor | None = None  # [rows, 512] latent dims (the GEMM input)
        if reserve_scratch:
            self._prefill_scratch(prefill_scratch_rows)
            self._eager_workspace(2 * self.num_ctas)

    # ------------------------------------------------------------------ workspace
    def _new_workspace(self, slots: int) -> Tuple[torch.Tensor, torch.Tensor]:
        capturing = torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
        assert not capturing, "decode workspaces are allocated outside capture"
        assert self.config.kv_lora_rank == 512
        return lib.decode_workspace(slots, self.num_heads, self.device)

    def _eager_workspace(self, slots: int) -> Tuple[torch.Tensor, torch.Tensor]:
        if self.ws_eager is None or self.ws_eager[0].shape[0] < slots:
            if self.ws_eager is not None and self.ws_eager_fence is not None:
                self.ws_retired.append((self.ws_eager, self.ws_eager_fence))
            self.ws_eager = self._new_workspace(max(slots, 2 * self.num_ctas))
            self.ws_eager_fence = None
        # drop retired workspaces whose last decode has completed
        self.ws_retired = [(ws, ev) for ws, ev in self.ws_retired if not ev.query()]
        return self.ws_eager

    # ------------------------------------------------------------------ forward
    def register_kv_b(self, layer_id: int, kv_b: torch.Tensor) -> None:
        """The decompression weight of layer ``layer_id``: ``kv_b [H * (128 + 128), 512]`` bf16, head
        h's rows ``256h .. 256h + 127`` give its k_nope, the next 128 its v (DeepSeek-V3's
        ``kv_b_proj`` layout). Prefill batches of that layer decompress the latent keys with it."""
        H = self.num_heads
        assert kv_b.shape == (H * 256, self.config.kv_lora_rank) and kv_b.dtype == torch.bfloat16
        self.kv_b[layer_id] = kv_b

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, layer_id: int, batch: Batch) -> torch.Tensor:
        """``k [T, 576]``: the new tokens' latent rows (``v`` unused: the values are their first 512
        dims), stored into the pool; then decode (``q [B, H, 576]``) or prefill (``q [T, H, 192]``)."""
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
        if self.ws_eager is not None and ws_o is self.ws_eager[0] and not torch.cuda.is_current_stream_capturing():
            if self.ws_eager_fence is None:
                self.ws_eager_fence = torch.cuda.Event()
            self.ws_eager_fence.record()  # on the current (engine) stream, after this decode
        self.last_lse = lse
        return out

    def _prefill_scratch(self, rows: int) -> Tuple[torch.Tensor, torch.Tensor]:
        if self.scratch_rows is None or self.scratch_rows.shape[0] < rows:
            n = max(rows, min(self.prefill_scratch_rows, 4 * rows))
            n = -(-n // PREFILL_PAGE) * PREFILL_PAGE
            self.scratch_rows = self.scratch_c = None
            H, dev = self.num_heads, self.device
            self.scratch_rows = torch.empty((n, H * 256 + 64), dtype=torch.bfloat16, device=dev)
            self.scratch_c = torch.empty((n, self.config.kv_lora_rank), dtype=torch.bfloat16, device=dev)
        return self.scratch_rows, self.scratch_c

    def _forward_prefill(self, q: torch.Tensor, layer_id: int, md: MLAMetadata) -> torch.Tensor:
        """Chunked prefill from the latent pool: ``q [T, H, 192]`` -> ``[T, H, 128]``.

        Per pass of whole requests: the latent rows of every key (prefix and chunk, already in the
        pool) are gathered into 64-token scratch pages (HIP, bit-exact), decompressed per head by one
        GEMM ``[k_nope | v] = c W_kvb^T`` (hipBLASLt) into the same scratch rows, whose tail keeps the
        key's shared rope dims; the prefill kernel then attends every request's prefix and itself
        causally (bottom-right aligned, ``attention/fa.py:155``) over those pages."""
        kv_b = self.kv_b.get(layer_id)
        if kv_b is None:
            raise lib.MLAKernelError(f"layer {layer_id}: no W_kvb registered (register_kv_b) for prefill")
        T, H, _ = q.shape
        out = torch.empty((T, H, self.config.v_head_dim), dtype=q.dtype, device=q.device)
        lse = torch.empty((T, H), dtype=torch.float32, device=q.device)
        pool = self.kvcache.latent_cache(layer_id)
        need = max(p[2] for p in md.prefill_plan)
        srows, sc = self._prefill_scratch(need)
        width = H * 256
        for r0, r1, rows, max_pages, off, q_rows in md.prefill_plan:
            n = r1 - r0
            seg_pt = md.prefill_seg_pt[r0:r1]
            lib.prefill_gather(pool, md.page_table[r0:r1], md.cache_seqlens[r0:r1], md.prefill_seg_first[off : off + n],
                               max_pages, sc[:rows], srows[:rows, width:], seg_pt)
            torch.mm(sc[:rows], kv_b.t(), out=srows[:rows, :width])
            lib.mla_prefill_decompressed(q, srows[:rows], seg_pt, md.cu_seqlens_q[r0 : r1 + 1],
                                         md.cache_seqlens[r0:r1], q_rows, self.scale, out, lse)
        self.last_lse = lse
        return out

    def _plan(self, seqlens_k: List[int], grid: int | None = None):
        """Split plan on the smallest grid of ``num_ctas * 2^k`` CTAs that holds the batch (one CTA per
        compute unit unless a CTA's range would pass the kernels' per-CTA limits of
        ``MAX_CTA_BLOCKS`` blocks or ``MAX_CTA_REQUESTS`` requests; further CTAs run as further
        rounds). With ``grid`` the plan is laid out for a launch of ``grid`` CTAs: the CTAs past the
        planned ones get empty ranges. Returns ``(plan, slots, launch CTAs)``."""
        ctas = self.num_ctas
        limit = grid if grid is not None else max(self.num_ctas, plan_grid_bound(self.num_ctas, sum(seqlens_k), len(seqlens_k)))
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
        prefill_plan = seg_first_dev = seg_pt = None
        if not is_decode:
            prefill_plan, firsts = [], []
            max_pages_all = 0
            for r0, r1, first in prefill_passes(seqlens_k, self.prefill_scratch_rows):
                pages = [-(-L // PREFILL_PAGE) for L in seqlens_k[r0:r1]]
                rows = (first[-1] + pages[-1]) * PREFILL_PAGE
                max_pages = max(max(pages), 1)
                max_pages_all = max(max_pages_all, max_pages)
                prefill_plan.append((r0, r1, max(rows, PREFILL_PAGE), max_pages, len(firsts), sum(seqlens_q[r0:r1])))
                firsts += first
            seg_first_dev = torch.tensor(firsts, **_CPU_I32).to(device, non_blocking=True)
            seg_pt = torch.empty((padded_size, max_pages_all), dtype=torch.int32, device=device)
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
            num_ctas=ctas if is_decode else 0,
            workspace=workspace,
            prefill_plan=prefill_plan,
            prefill_seg_first=seg_first_dev,
            prefill_seg_pt=seg_pt,
        )

    # ------------------------------------------------------------------ graph capture
    def init_capture_graph(self, max_seq_len: int, bs_list: List[int]) -> None:
        assert self.capture is None, "Capture already initialized."
        max_bs = max(bs_list)
        cols = -(-max_seq_len // self.page_size)
        # the captured launch has a fixed plan grid: the one the largest batch the graphs can replay
        # needs. Its tokens are bounded by max_bs * max_seq_len, not by the pool: requests sharing
        # prefix pages (the radix cache) can hold more tokens in all than the pool has. The kernels
        # run a plan of more ranges than compute units as a loop over ranges (the launch grid stays
        # at one CTA per compute unit) and stop at the first padding range, so a large plan grid costs
        # only its workspace (2 slots per range)
        self.capture_ctas = plan_grid_bound(self.num_ctas, max_bs * max_seq_len, max_bs)
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
