"""CPU oracle for the MLA attention hot path.

TEST INFRASTRUCTURE ONLY. This module is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The product path (``minisgl_amd``) never calls it, and fails loudly
when its HIP library is missing instead of falling back here.

What it restates, and from where:

* ``page_table_from_tokens`` -- the token-to-page table conversion of the
  reference's attention backends, ``python/minisgl/attention/fa.py:92-97``
  (identical in ``attention/trtllm.py:116-121``). The source table is
  ``Context.page_table`` (``python/minisgl/core.py:103-104``), which holds one
  token location per column ("always treat page_size = 1").
* ``store_rows`` -- the KV scatter ``cache[indices[i]] = x[i]`` of
  ``python/minisgl/kernel/csrc/jit/store.cu:25-53`` as used by
  ``MHAKVCache.store_kv`` (``python/minisgl/kvcache/mha_pool.py:45-56``).
* ``gather_rows`` -- the paged read every attention kernel performs: token
  ``t`` of a request lives at row ``page_table[t // ps] * ps + t % ps`` of the
  flattened pool (layout of ``kvcache/mha_pool.py:28-32``; page ids produced by
  ``scheduler/cache.py:119-146``).
* ``mla_decode`` / ``mla_decode_pieces`` / ``mla_merge`` -- absorbed-MLA decode
  and its split-KV log-sum-exp merge. The reference has no MLA code
  (``kvcache/__init__.py:34`` is a TODO; ``models/register.py:5-12`` lists no
  DeepSeek/Kimi model) and its attention arithmetic lives in un-vendored
  CUDA-only packages (``attention/fa.py:157-182``, ``attention/fi.py:134-188``),
  so these follow the mathematics: per (request, head)
  ``s_t = scale * <q, kv_t>``, ``o = sum_t softmax(s)_t * kv_t[:dv]``,
  ``lse = ln sum_t exp(s_t)`` (natural log). The masking convention is the
  reference's ``causal=True`` with bottom-right alignment
  (``attention/fa.py:155``): a decode query sees all ``device_len`` tokens.
* ``mla_prefill`` -- chunked (extend) prefill over a paged prefix, causal with
  bottom-right alignment: query ``i`` of a request with ``L`` total and ``E``
  new tokens sits at absolute position ``L - E + i`` and sees keys ``j <= L -
  E + i`` (``attention/fa.py:84-90,155``; lengths from ``core.py:44-50``).
* ``decompress_pool`` -- per-head K/V of latent rows, the decompression the MLA
  layer does before a chunked prefill (the caller role of
  ``layers/attention.py:47-57``, MLA having no code in the reference): with
  ``W_kvb [H * 256, 512]`` (head ``h``'s rows ``256h .. 256h + 127`` give its
  k_nope, the next 128 its v), ``K[t, h] = [W_kvb[256h : 256h+128] c_t | k_pe_t]``
  and ``V[t, h] = W_kvb[256h+128 : 256h+256] c_t``.

Empty inputs: a request with zero keys yields ``o = 0`` and ``lse = -inf``.

Pins (tests/test_oracle.py): float64 pure-Python loops on tiny inputs, the
closed forms (one key, equal scores, dominant key, score shift), torch's
``scaled_dot_product_attention`` on CPU, split/merge equivalence, the
absorbed-vs-decompressed MLA identity (through ``decompress_pool``), scalar loops
for ``decompress_pool`` and the reference's own bit-exact store
and page-table invariants (``tests/kernel/test_store.py:33-34``,
``tests/core/test_cache_allocate.py:147-169``).
"""

from __future__ import annotations

import math
from typing import List, Sequence, Tuple

import torch

LATENT_DIM = 512
ROPE_DIM = 64
KV_DIM = LATENT_DIM + ROPE_DIM  # 576
PREFILL_QK_DIM = 192  # 128 nope + 64 rope
PREFILL_V_DIM = 128
DEFAULT_SCALE = 1.0 / math.sqrt(PREFILL_QK_DIM)


def page_table_from_tokens(
    token_table: torch.Tensor, table_idx: torch.Tensor, max_seqlen_k: int, page_size: int
) -> torch.Tensor:
    """``new_pt[b, j] = token_table[table_idx[b], j * ps] // ps``.

    Restates ``python/minisgl/attention/fa.py:92-97``: the columns are the
    token-table slice ``[: max_seqlen_k : page_size]`` (``ceil(max_seqlen_k /
    ps)`` of them), floor-divided by the page size when it exceeds one.
    """
    rows = token_table[table_idx.long()]
    sliced = rows[:, :max_seqlen_k:page_size]
    if page_size > 1:
        return torch.div(sliced, page_size, rounding_mode="floor").to(torch.int32)
    return sliced.to(torch.int32).clone()


def store_rows(cache: torch.Tensor, indices: torch.Tensor, x: torch.Tensor) -> None:
    """``cache[indices[i], :] = x[i, :]`` (``kernel/csrc/jit/store.cu:41-49``)."""
    cache[indices.long()] = x


def token_rows(page_table_row: torch.Tensor, length: int, page_size: int) -> torch.Tensor:
    """Flattened pool row of each of the first ``length`` tokens of one request."""
    t = torch.arange(length, dtype=torch.int64)
    pages = page_table_row.long()[t // page_size]
    return pages * page_size + t % page_size


def decompress_pool(latent_pool: torch.Tensor, kv_b: torch.Tensor, num_heads: int, out_dtype=None):
    """Per-head pages ``K [pages, ps, H, 192]``, ``V [pages, ps, H, 128]`` of a latent pool
    ``[pages, ps, 576]`` with ``kv_b [H * 256, 512]`` (float32 math, float64 for float64 inputs);
    ``out_dtype`` rounds K and V to it (the GPU path writes bf16 decompressed rows)."""
    dt = torch.float64 if latent_pool.dtype == torch.float64 else torch.float32
    pages, ps, _ = latent_pool.shape
    rows = latent_pool.reshape(-1, KV_DIM).to(dt)
    w = kv_b.to(dt).view(num_heads, 2, 128, LATENT_DIM)  # [head][k_nope | v][dim][latent]
    kv = torch.einsum("tl,hjdl->thjd", rows[:, :LATENT_DIM], w)  # [rows, H, 2, 128]
    k = torch.cat([kv[:, :, 0], rows[:, None, LATENT_DIM:].expand(-1, num_heads, -1)], dim=-1)
    v = kv[:, :, 1]
    if out_dtype is not None:
        k, v = k.to(out_dtype), v.to(out_dtype)
    return k.reshape(pages, ps, num_heads, PREFILL_QK_DIM), v.reshape(pages, ps, num_heads, PREFILL_V_DIM)


def gather_rows(pool_flat: torch.Tensor, page_table_row: torch.Tensor, length: int, page_size: int):
    """Rows ``[0, length)`` of one request from a pool flattened to ``[pages*ps, ...]``."""
    return pool_flat[token_rows(page_table_row, length, page_size)]


def _attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, mask=None):
    """Softmax attention of ``q [H, M, D]`` over ``k [H, N, D]`` / ``v [H, N, Dv]``.

    Returns ``o [H, M, Dv]`` and natural-log ``lse [H, M]``; a row with no
    visible key gives ``o = 0`` and ``lse = -inf``.
    """
    s = torch.matmul(q, k.transpose(-1, -2)) * scale
    if mask is not None:
        s = s.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    finite = torch.isfinite(lse)
    p = torch.exp(s - torch.where(finite, lse, torch.zeros_like(lse)).unsqueeze(-1))
    p = torch.where(finite.unsqueeze(-1), p, torch.zeros_like(p))
    o = torch.matmul(p, v)
    return o, lse


def mla_decode(
    q: torch.Tensor,
    kv_pool: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: Sequence[int] | torch.Tensor,
    scale: float = DEFAULT_SCALE,
    *,
    dv: int = LATENT_DIM,
    dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Absorbed-MLA paged decode.

    ``q [B, H, Dk]`` (Dk = 576), ``kv_pool [pages, ps, Dk]`` latent cache whose
    value is its first ``dv`` dims, ``page_table [B, >= ceil(L/ps)]`` page ids,
    ``seq_lens [B]`` = ``device_len`` (includes the token being decoded).
    Returns ``o [B, H, dv]`` and ``lse [B, H]`` in ``dtype``.
    """
    B, H, D = q.shape
    ps = kv_pool.shape[1]
    flat = kv_pool.reshape(-1, kv_pool.shape[-1])
    lens = [int(x) for x in seq_lens]
    o = torch.zeros((B, H, dv), dtype=dtype)
    lse = torch.full((B, H), float("-inf"), dtype=dtype)
    for b in range(B):
        if lens[b] == 0:
            continue
        kv = gather_rows(flat, page_table[b], lens[b], ps).to(dtype)  # [L, D]
        ob, lb = _attend(q[b].to(dtype).unsqueeze(1), kv.unsqueeze(0), kv[:, :dv].unsqueeze(0), scale)
        o[b] = ob[:, 0]
        lse[b] = lb[:, 0]
    return o, lse


def mla_decode_pieces(
    q: torch.Tensor,
    kv_pool: torch.Tensor,
    page_table: torch.Tensor,
    pieces: List[Tuple[int, int, int]],
    scale: float = DEFAULT_SCALE,
    *,
    dv: int = LATENT_DIM,
    dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Attention of request ``b`` over its tokens ``[t0, t1)`` for each piece.

    Returns per-piece normalised ``o [N, H, dv]`` and ``lse [N, H]``: the
    partial results a split-KV decode produces before the merge.
    """
    H = q.shape[1]
    ps = kv_pool.shape[1]
    flat = kv_pool.reshape(-1, kv_pool.shape[-1])
    o = torch.zeros((len(pieces), H, dv), dtype=dtype)
    lse = torch.full((len(pieces), H), float("-inf"), dtype=dtype)
    for n, (b, t0, t1) in enumerate(pieces):
        if t1 <= t0:
            continue
        kv = gather_rows(flat, page_table[b], t1, ps)[t0:t1].to(dtype)
        ob, lb = _attend(q[b].to(dtype).unsqueeze(1), kv.unsqueeze(0), kv[:, :dv].unsqueeze(0), scale)
        o[n] = ob[:, 0]
        lse[n] = lb[:, 0]
    return o, lse


def mla_merge(o_parts: torch.Tensor, lse_parts: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Log-sum-exp merge of ``S`` normalised partials along dim 0.

    ``lse = ln sum_i exp(lse_i)``; ``o = sum_i exp(lse_i - lse) * o_i``. All
    partials empty (every ``lse_i = -inf``) gives ``o = 0``, ``lse = -inf``.
    """
    lse = torch.logsumexp(lse_parts, dim=0)
    finite = torch.isfinite(lse)
    w = torch.exp(lse_parts - torch.where(finite, lse, torch.zeros_like(lse)).unsqueeze(0))
    w = torch.where(finite.unsqueeze(0), w, torch.zeros_like(w))
    o = (w.unsqueeze(-1) * o_parts).sum(dim=0)
    return o, lse


def mla_prefill(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    page_table: torch.Tensor,
    cu_seqlens_q: Sequence[int] | torch.Tensor,
    seq_lens_k: Sequence[int] | torch.Tensor,
    scale: float = DEFAULT_SCALE,
    *,
    dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Chunked (extend) prefill over a paged prefix, causal, bottom-right aligned.

    ``q [T, H, Dqk]`` packed by ``cu_seqlens_q [B+1]``; ``k_pool [pages, ps, H,
    Dqk]``, ``v_pool [pages, ps, H, Dv]``; ``seq_lens_k [B]`` is the total
    length (prefix + extend) whose K/V are already in the pools. Returns ``o
    [T, H, Dv]`` and ``lse [T, H]``.
    """
    T, H, _ = q.shape
    ps = k_pool.shape[1]
    dv = v_pool.shape[-1]
    kflat = k_pool.reshape(-1, H, k_pool.shape[-1])
    vflat = v_pool.reshape(-1, H, dv)
    cu = [int(x) for x in cu_seqlens_q]
    lens = [int(x) for x in seq_lens_k]
    o = torch.zeros((T, H, dv), dtype=dtype)
    lse = torch.full((T, H), float("-inf"), dtype=dtype)
    for b in range(len(lens)):
        q0, q1 = cu[b], cu[b + 1]
        E, L = q1 - q0, lens[b]
        if E == 0:
            continue
        assert L >= E, "extend longer than the total length"
        rows = token_rows(page_table[b], L, ps)
        k = kflat[rows].to(dtype).transpose(0, 1)  # [H, L, D]
        v = vflat[rows].to(dtype).transpose(0, 1)
        qb = q[q0:q1].to(dtype).transpose(0, 1)  # [H, E, D]
        i = torch.arange(E).unsqueeze(1) + (L - E)
        j = torch.arange(L).unsqueeze(0)
        ob, lb = _attend(qb, k, v, scale, mask=(j <= i).unsqueeze(0))
        o[q0:q1] = ob.transpose(0, 1)
        lse[q0:q1] = lb.transpose(0, 1)
    return o, lse
