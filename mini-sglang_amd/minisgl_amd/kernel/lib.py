"""ctypes binding of libmla_amd.so (C ABI declared in include/mla_amd.h).

The library is required: every entry here raises if it is missing or a call
fails, mirroring the reference's RuntimeCheck -> Python exception path
(python/minisgl/kernel/csrc/include/minisgl/utils.h:40-93). There is no
fallback implementation.
"""

from __future__ import annotations

import ctypes
import functools
import os
from typing import Tuple

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmla_amd.so")

_c_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32

# symbol -> (restype, argtypes); must match include/mla_amd.h
SIGNATURES = {
    "mla_last_error": (ctypes.c_char_p, []),
    "mla_abi_version": (ctypes.c_int, []),
    "mla_device_cu_count": (ctypes.c_int, [ctypes.c_int, _c_i32p]),
    "mla_store_rows": (ctypes.c_int, [_vp, _i64, _i64, _vp, _i64, _vp, _i32, _i64, _i64, _vp]),
    "mla_prefill_gather_bf16": (
        ctypes.c_int,
        [_vp, _i64, _i32, _i32, _vp, _i64, _vp, _vp, _i32, _i32, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp],
    ),
    "mla_page_table_from_tokens": (
        ctypes.c_int,
        [_vp, _i32, _i32, _i64, _vp, _i32, _i32, _i32, _vp, _i64, _vp],
    ),
    "mla_decode_plan": (ctypes.c_int, [_c_i32p, _i32, _i32, _i32, _i32, _c_i32p, _c_i32p, _c_i32p]),
    "mla_decode_bf16": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _i64, _i32, _i32, _vp, _i64, _vp, _i32, _i32, ctypes.c_float, _vp, _i32,
         _vp, _vp, _i32, _vp, _i64, _i64, _vp, _i64, _vp],
    ),
    "mla_decode_split_bf16": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _i64, _i32, _i32, _vp, _i64, _vp, _i32, _i32, ctypes.c_float, _vp, _i32,
         _vp, _vp, _i32, _vp, _i64, _i64, _vp, _i64, _vp],
    ),
    "mla_decode_bf16_noalloc": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _i64, _i32, _i32, _vp, _i64, _vp, _i32, _i32, ctypes.c_float, _vp, _i32, _i32,
         _vp, _i64, _i64, _vp, _i64, _vp],
    ),
    "mla_decode_merge_f32": (
        ctypes.c_int, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp, _i64, _i64, _vp, _i64, _vp]
    ),
    "mla_prefill_bf16": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _i64, _vp, _i64, _i32, _i32, _vp, _i64, _vp, _vp, _i32, _i32, _i32, ctypes.c_float,
         _vp, _i64, _i64, _vp, _i64, _vp],
    ),
    "mla_prefill_strided_bf16": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _i32, _vp, _i64, _vp, _vp, _i32, _i32,
         _i32, ctypes.c_float, _vp, _i64, _i64, _vp, _i64, _vp],
    ),
    "mla_rmsnorm_bf16": (ctypes.c_int, [_vp, _i64, _vp, _i32, _i32, ctypes.c_float, _vp, _i64, _vp]),
    "mla_latent_rows_bf16": (
        ctypes.c_int, [_vp, _i64, _vp, _vp, _vp, _i32, _i32, ctypes.c_float, _i32, _vp, _i64, _vp]
    ),
    "mla_qkv_a_rows_bf16": (
        ctypes.c_int, [_vp, _i64, _i32, _vp, _vp, _vp, _vp, _i32, _i32, ctypes.c_float, _i32, _vp, _i64, _vp]
    ),
    "mla_q_rope_bf16": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i32, _i32, _vp, _vp, _i32, _i32, _vp, _i64, _i64, _vp, _i64, _i64, _vp],
    ),
}

ABI_VERSION = 9
PLAN_BLOCK = 64
PLAN_CTA_INTS = 4
PLAN_REQ_INTS = 3
MAX_CTA_BLOCKS = 512
MAX_CTA_REQUESTS = 128


def partial_chunk_dims():
    """Value dim held at each of the 512 positions of a split-KV partial row (the chunk order of
    ``include/mla_amd.h``): 16-byte chunk c holds dims 32 (c // 4) + 4 (c % 4) + {0..3}, then the
    same + 16."""
    c = np.arange(64)[:, None]
    e = np.arange(8)[None, :]
    return (32 * (c // 4) + 4 * (c % 4) + (e % 4) + 16 * (e // 4)).reshape(-1)


def decode_workspace(slots: int, heads: int, device):
    """Split-KV workspace for ``slots`` partial slots: ``ws_o [slots, heads, 512]`` bf16 and
    ``ws_lse [slots, heads]`` fp32 (at least one slot, so the pointers are valid)."""
    import torch

    n = max(int(slots), 1)
    return (torch.empty((n, heads, 512), dtype=torch.bfloat16, device=device),
            torch.empty((n, heads), dtype=torch.float32, device=device))


class MLAKernelError(RuntimeError):
    """A libmla_amd entry point returned an error code."""


@functools.lru_cache(maxsize=None)
def load_library() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise MLAKernelError(
            f"{LIB_PATH} is missing: build it with `python mini-sglang_amd/build.py` "
            "(the MLA backend has no non-HIP fallback)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.mla_abi_version() != ABI_VERSION:
        raise MLAKernelError(f"libmla_amd ABI {lib.mla_abi_version()} != expected {ABI_VERSION}")
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_library().mla_last_error().decode(errors="replace")
        raise MLAKernelError(f"{what} failed (code {rc}): {msg}")


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int | None:
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def device_cu_count(device: int = 0) -> int:
    out = ctypes.c_int32(0)
    check(load_library().mla_device_cu_count(device, ctypes.byref(out)), "mla_device_cu_count")
    return int(out.value)


def store_rows(cache, indices, x, stream=None) -> None:
    """``cache[indices[i]] = x[i]`` over the leading dim; rows are the remaining dims."""
    import torch

    assert cache.is_cuda and x.is_cuda and indices.is_cuda, "store_rows needs device tensors"
    assert cache.dtype == x.dtype, "cache and x dtypes differ"
    n = x.shape[0]
    row_bytes = x[0].numel() * x.element_size() if n else cache[0].numel() * cache.element_size()
    assert cache[0].numel() * cache.element_size() == row_bytes, "row widths differ"
    assert indices.dim() == 1 and indices.shape[0] == n and indices.dtype in (torch.int32, torch.int64)
    x2 = x.reshape(n, -1) if n else x
    c2 = cache.view(cache.shape[0], -1)
    assert x2.stride(-1) == 1 and c2.stride(-1) == 1, "rows must be contiguous"
    check(
        load_library().mla_store_rows(
            _ptr(c2), c2.shape[0], c2.stride(0) * c2.element_size(), _ptr(x2),
            (x2.stride(0) if n else row_bytes // x.element_size()) * x.element_size(), _ptr(indices),
            32 if indices.dtype == torch.int32 else 64, n, row_bytes, _stream(stream),
        ),
        "mla_store_rows",
    )


def page_table_from_tokens(token_table, table_idx, max_seqlen_k: int, page_size: int, out=None, stream=None):
    """Device page table ``[B, ceil(max_seqlen_k / ps)]`` from the token-level table."""
    import torch

    assert token_table.dtype == torch.int32 and table_idx.dtype == torch.int32
    assert token_table.stride(-1) == 1
    B = table_idx.shape[0]
    cols = -(-max_seqlen_k // page_size)
    if out is None:
        out = torch.empty((B, cols), dtype=torch.int32, device=token_table.device)
    check(
        load_library().mla_page_table_from_tokens(
            _ptr(token_table), token_table.shape[0], token_table.shape[1], token_table.stride(0),
            _ptr(table_idx), B, max_seqlen_k, page_size, _ptr(out), out.stride(0), _stream(stream),
        ),
        "mla_page_table_from_tokens",
    )
    return out


def decode_plan(
    seq_lens, page_size: int, num_ctas: int, max_piece_pages: int = 0
) -> Tuple[np.ndarray, int]:
    """Host split-KV plan: int32 ``[num_ctas*4 + B*3]`` (CTA ranges, then request info), slots.
    ``max_piece_pages > 0`` caps the pages one piece touches (0: pieces of any length)."""
    lens = np.ascontiguousarray(np.asarray(seq_lens, dtype=np.int32))
    B = int(lens.shape[0])
    plan = np.zeros(num_ctas * PLAN_CTA_INTS + B * PLAN_REQ_INTS, dtype=np.int32)
    slots = ctypes.c_int32(0)
    cta = plan[: num_ctas * PLAN_CTA_INTS]
    req = plan[num_ctas * PLAN_CTA_INTS :]
    p32 = lambda a: a.ctypes.data_as(_c_i32p)  # noqa: E731
    check(
        load_library().mla_decode_plan(
            p32(lens), B, page_size, num_ctas, max_piece_pages, p32(cta),
            p32(req) if B else None, ctypes.byref(slots),
        ),
        "mla_decode_plan",
    )
    return plan, int(slots.value)


def mla_decode(
    q, kv_pool, page_table, seq_lens, plan, num_ctas: int, ws_o, ws_lse, scale: float, out, lse=None,
    stream=None, split_only: bool = False,
) -> None:
    """Absorbed-MLA decode: ``q [B, H, 576]``, ``kv_pool [pages, ps, 576]`` -> ``out [B, H, 512]``.

    ``split_only`` launches just the split kernel (partials stay in the
    workspace for ``mla_decode_merge(..., single_piece_final=True)``).
    """
    import torch

    B, H, D = q.shape
    assert D == 576 and kv_pool.shape[-1] == 576 and q.dtype == torch.bfloat16 and kv_pool.dtype == torch.bfloat16
    assert q.stride(-1) == 1 and kv_pool.stride(-1) == 1
    assert kv_pool.stride(0) == kv_pool.shape[1] * kv_pool.stride(1), "pool pages must be row-contiguous"
    assert page_table.dtype == torch.int32 and seq_lens.dtype == torch.int32 and plan.dtype == torch.int32
    assert out.shape == (B, H, 512) and out.dtype == torch.bfloat16 and out.stride(-1) == 1
    assert plan.numel() >= num_ctas * PLAN_CTA_INTS + B * PLAN_REQ_INTS
    ws_slots = 0 if ws_o is None else ws_o.shape[0]
    if ws_o is not None:
        assert ws_o.shape[1:] == (H, 512) and ws_lse.shape[:2] == (ws_slots, H)
        assert ws_o.dtype == torch.bfloat16 and ws_lse.dtype == torch.float32, "ws_o is bf16, ws_lse fp32"
    if lse is not None:
        assert lse.dtype == torch.float32 and lse.shape == (B, H) and lse.stride(-1) == 1
    fn = load_library().mla_decode_split_bf16 if split_only else load_library().mla_decode_bf16
    check(
        fn(
            _ptr(q), q.stride(0), q.stride(1), _ptr(kv_pool), kv_pool.stride(1),
            kv_pool.shape[0], kv_pool.shape[1], _ptr(page_table), page_table.stride(0), _ptr(seq_lens), B, H,
            float(scale), _ptr(plan), num_ctas, _ptr(ws_o), _ptr(ws_lse), ws_slots, _ptr(out), out.stride(0),
            out.stride(1), _ptr(lse), 0 if lse is None else lse.stride(0), _stream(stream),
        ),
        "mla_decode_split_bf16" if split_only else "mla_decode_bf16",
    )


NOALLOC_MAX_SLOT_HEADS = 32768


def mla_decode_noalloc(q, kv_pool, page_table, seq_lens, plan, num_ctas: int, num_slots: int, scale: float, out,
                       lse=None, stream=None) -> None:
    """``mla_decode`` with the split-KV partials in the library's fixed scratch (no workspace):
    ``num_slots`` is the plan's slot count; calls that overlap on one GPU race."""
    import torch

    B, H, D = q.shape
    assert D == 576 and kv_pool.shape[-1] == 576 and q.dtype == torch.bfloat16 and kv_pool.dtype == torch.bfloat16
    assert q.stride(-1) == 1 and kv_pool.stride(-1) == 1
    assert kv_pool.stride(0) == kv_pool.shape[1] * kv_pool.stride(1), "pool pages must be row-contiguous"
    assert page_table.dtype == torch.int32 and seq_lens.dtype == torch.int32 and plan.dtype == torch.int32
    assert out.shape == (B, H, 512) and out.dtype == torch.bfloat16 and out.stride(-1) == 1
    assert plan.numel() >= num_ctas * PLAN_CTA_INTS + B * PLAN_REQ_INTS
    if lse is not None:
        assert lse.dtype == torch.float32 and lse.shape == (B, H) and lse.stride(-1) == 1
    check(
        load_library().mla_decode_bf16_noalloc(
            _ptr(q), q.stride(0), q.stride(1), _ptr(kv_pool), kv_pool.stride(1),
            kv_pool.shape[0], kv_pool.shape[1], _ptr(page_table), page_table.stride(0), _ptr(seq_lens), B, H,
            float(scale), _ptr(plan), num_ctas, num_slots, _ptr(out), out.stride(0), out.stride(1), _ptr(lse),
            0 if lse is None else lse.stride(0), _stream(stream),
        ),
        "mla_decode_bf16_noalloc",
    )


def mla_decode_merge(ws_o, ws_lse, req_info, out, lse=None, stream=None, single_piece_final: bool = False) -> None:
    """fp32 LSE merge of partials ``ws_o [S, H, 512]`` (bf16, chunk order of ``partial_chunk_dims``) /
    ``ws_lse [S, H]`` (fp32) per ``req_info``."""
    import torch

    assert ws_o.dtype == torch.bfloat16 and ws_lse.dtype == torch.float32, "ws_o is bf16, ws_lse fp32"
    B, H = out.shape[0], out.shape[1]
    check(
        load_library().mla_decode_merge_f32(
            _ptr(ws_o), _ptr(ws_lse), ws_o.shape[0], _ptr(req_info), B, H, int(single_piece_final), _ptr(out),
            out.stride(0), out.stride(1),
            _ptr(lse), 0 if lse is None else lse.stride(0), _stream(stream),
        ),
        "mla_decode_merge_f32",
    )


def mla_prefill(q, k_pool, v_pool, page_table, cu_seqlens_q, seq_lens_k, scale: float, out, lse=None,
                stream=None) -> None:
    """Chunked MLA prefill: ``q [T, H, 192]``, ``k_pool [pages, ps, H, 192]``, ``v_pool [pages, ps, H, 128]``
    -> ``out [T, H, 128]`` (+ ``lse [T, H]``); causal over each request's prefix + extend."""
    import torch

    T, H, D = q.shape
    assert D == 192 and q.dtype == torch.bfloat16 and q.stride(-1) == 1
    assert k_pool.dim() == 4 and k_pool.shape[2:] == (H, 192) and v_pool.shape[2:] == (H, 128)
    assert k_pool.dtype == torch.bfloat16 and v_pool.dtype == torch.bfloat16
    assert k_pool.stride(3) == 1 and k_pool.stride(2) == 192 and v_pool.stride(3) == 1 and v_pool.stride(2) == 128
    assert k_pool.stride(0) == k_pool.shape[1] * k_pool.stride(1) and v_pool.stride(0) == v_pool.shape[1] * v_pool.stride(1)
    assert k_pool.shape[:2] == v_pool.shape[:2]
    assert page_table.dtype == torch.int32 and cu_seqlens_q.dtype == torch.int32 and seq_lens_k.dtype == torch.int32
    assert out.shape == (T, H, 128) and out.dtype == torch.bfloat16 and out.stride(-1) == 1
    B = seq_lens_k.shape[0]
    assert cu_seqlens_q.shape[0] == B + 1
    if lse is not None:
        assert lse.dtype == torch.float32 and lse.shape == (T, H) and lse.stride(-1) == 1
    check(
        load_library().mla_prefill_bf16(
            _ptr(q), q.stride(0), q.stride(1), _ptr(k_pool), k_pool.stride(1), _ptr(v_pool), v_pool.stride(1),
            k_pool.shape[0], k_pool.shape[1], _ptr(page_table), page_table.stride(0), _ptr(cu_seqlens_q),
            _ptr(seq_lens_k), B, T, H, float(scale), _ptr(out), out.stride(0), out.stride(1), _ptr(lse),
            0 if lse is None else lse.stride(0), _stream(stream),
        ),
        "mla_prefill_bf16",
    )


def mla_prefill_strided(q, k_nope, k_row_stride: int, k_head_stride: int, k_rope, k_rope_head_stride: int, v,
                        v_row_stride: int, v_head_stride: int, num_pages: int, page_size: int, page_table,
                        cu_seqlens_q, seq_lens_k, total_q: int, scale: float, out, lse=None, stream=None) -> None:
    """``mla_prefill`` with K and V rows anywhere (``mla_prefill_strided_bf16``): ``k_nope``,
    ``k_rope`` and ``v`` are bf16 tensors whose first elements are those of token row 0 / head 0;
    strides in elements; token row r = page * page_size + offset. ``total_q`` bounds the launch
    (at least the query rows of this batch)."""
    import torch

    T, H, D = q.shape
    assert D == 192 and q.dtype == torch.bfloat16 and q.stride(-1) == 1
    for t in (k_nope, k_rope, v):
        assert t.dtype == torch.bfloat16 and t.is_cuda
    assert page_table.dtype == torch.int32 and cu_seqlens_q.dtype == torch.int32 and seq_lens_k.dtype == torch.int32
    assert out.shape == (T, H, 128) and out.dtype == torch.bfloat16 and out.stride(-1) == 1
    B = seq_lens_k.shape[0]
    assert cu_seqlens_q.shape[0] == B + 1
    if lse is not None:
        assert lse.dtype == torch.float32 and lse.shape == (T, H) and lse.stride(-1) == 1
    check(
        load_library().mla_prefill_strided_bf16(
            _ptr(q), q.stride(0), q.stride(1), _ptr(k_nope), k_row_stride, k_head_stride, _ptr(k_rope),
            k_rope_head_stride, _ptr(v), v_row_stride, v_head_stride, num_pages, page_size, _ptr(page_table),
            page_table.stride(0), _ptr(cu_seqlens_q), _ptr(seq_lens_k), B, total_q, H, float(scale), _ptr(out),
            out.stride(0), out.stride(1), _ptr(lse), 0 if lse is None else lse.stride(0), _stream(stream),
        ),
        "mla_prefill_strided_bf16",
    )


def mla_prefill_decompressed(q, rows, page_table, cu_seqlens_q, seq_lens_k, total_q: int, scale: float, out,
                             lse=None, stream=None) -> None:
    """Prefill over decompressed scratch rows ``rows [n, H * 256 + 64]`` (per key: head h's k_nope
    at ``256h``, its v at ``256h + 128``, the shared rope dims at ``256H``), in 64-row pages under
    ``page_table`` (``prefill_gather``'s scratch page table)."""
    H = q.shape[1]
    n, width = rows.shape
    assert width == 256 * H + 64 and rows.stride(1) == 1 and n % 64 == 0
    stride = rows.stride(0)
    mla_prefill_strided(q, rows, stride, 256, rows[:, 256 * H :], 0, rows[:, 128:], stride, 256, n // 64, 64,
                        page_table, cu_seqlens_q, seq_lens_k, total_q, scale, out, lse, stream)


def prefill_gather(kv_pool, page_table, seq_lens_k, seg_first, max_seg_pages: int, c_out, rope_out, seg_page_table,
                   stream=None) -> None:
    """``mla_prefill_gather_bf16``: key j of request b (pool ``kv_pool [pages, ps, 576]`` through
    ``page_table``) to scratch row ``64 seg_first[b] + j`` of ``c_out [rows, 512]`` (latent dims)
    and ``rope_out [rows, 64]`` (rope dims); ``seg_page_table[b, i] = seg_first[b] + i``."""
    import torch

    assert kv_pool.dim() == 3 and kv_pool.shape[-1] == 576 and kv_pool.dtype == torch.bfloat16
    assert kv_pool.stride(-1) == 1 and kv_pool.stride(0) == kv_pool.shape[1] * kv_pool.stride(1)
    assert c_out.shape[1] == 512 and rope_out.shape[1] == 64 and c_out.shape[0] == rope_out.shape[0]
    assert c_out.stride(1) == 1 and rope_out.stride(1) == 1
    for t in (page_table, seq_lens_k, seg_first, seg_page_table):
        assert t.dtype == torch.int32
    B = seq_lens_k.shape[0]
    assert seg_first.shape[0] >= B and seg_page_table.shape[0] >= B and seg_page_table.shape[1] >= max_seg_pages
    check(
        load_library().mla_prefill_gather_bf16(
            _ptr(kv_pool), kv_pool.stride(1), kv_pool.shape[0], kv_pool.shape[1], _ptr(page_table),
            page_table.stride(0), _ptr(seq_lens_k), _ptr(seg_first), B, max_seg_pages, _ptr(c_out), c_out.stride(0),
            _ptr(rope_out), rope_out.stride(0), c_out.shape[0], _ptr(seg_page_table), seg_page_table.stride(0),
            _stream(stream),
        ),
        "mla_prefill_gather_bf16",
    )


def rmsnorm(x, weight, eps: float, out=None, stream=None):
    """``x [rows, n]`` bf16 -> ``x / sqrt(mean(x^2) + eps) * weight`` (``out`` may be ``x``)."""
    import torch

    assert x.dim() == 2 and x.dtype == torch.bfloat16 and x.stride(1) == 1 and x.is_cuda
    rows, n = x.shape
    assert weight.shape == (n,) and weight.dtype == torch.bfloat16 and weight.is_contiguous()
    if out is None:
        out = torch.empty_like(x)
    assert out.shape == x.shape and out.dtype == torch.bfloat16 and out.stride(1) == 1
    check(
        load_library().mla_rmsnorm_bf16(_ptr(x), x.stride(0), _ptr(weight), rows, n, float(eps), _ptr(out),
                                        out.stride(0), _stream(stream)),
        "mla_rmsnorm_bf16",
    )
    return out


def latent_rows(kv, norm_weight, positions, cos_sin, eps: float, interleaved: bool, out=None, stream=None):
    """``kv [T, 576]`` (kv_a output) -> latent rows ``[T, 576]``: RMSNorm of the first 512 dims,
    RoPE of the last 64 at ``positions`` (int32) from the fp32 ``cos_sin [max_position, 64]`` table."""
    import torch

    assert kv.dim() == 2 and kv.shape[1] == 576 and kv.dtype == torch.bfloat16 and kv.stride(1) == 1 and kv.is_cuda
    T = kv.shape[0]
    assert norm_weight.shape == (512,) and norm_weight.dtype == torch.bfloat16 and norm_weight.is_contiguous()
    assert positions.shape == (T,) and positions.dtype == torch.int32 and positions.is_contiguous()
    assert cos_sin.dim() == 2 and cos_sin.shape[1] == 64 and cos_sin.dtype == torch.float32 and cos_sin.is_contiguous()
    if out is None:
        out = torch.empty((T, 576), dtype=torch.bfloat16, device=kv.device)
    assert out.shape == (T, 576) and out.dtype == torch.bfloat16 and out.stride(1) == 1
    check(
        load_library().mla_latent_rows_bf16(
            _ptr(kv), kv.stride(0), _ptr(norm_weight), _ptr(positions), _ptr(cos_sin), cos_sin.shape[0], T,
            float(eps), int(bool(interleaved)), _ptr(out), out.stride(0), _stream(stream),
        ),
        "mla_latent_rows_bf16",
    )
    return out


def q_rope(q, positions, cos_sin, interleaved: bool, pe_out, nope_out=None, stream=None) -> None:
    """``q [T, H, 192]``: ``pe_out [T, H, 64]`` = RoPE of the rope dims (may be ``q[..., 128:]``);
    ``nope_out [T, H, 128]`` (any strides, e.g. a head-major buffer's transpose) = the nope dims."""
    import torch

    assert q.dim() == 3 and q.shape[2] == 192 and q.dtype == torch.bfloat16 and q.stride(2) == 1 and q.is_cuda
    T, H, _ = q.shape
    assert positions.shape == (T,) and positions.dtype == torch.int32 and positions.is_contiguous()
    assert cos_sin.dim() == 2 and cos_sin.shape[1] == 64 and cos_sin.dtype == torch.float32 and cos_sin.is_contiguous()
    assert pe_out.shape == (T, H, 64) and pe_out.dtype == torch.bfloat16 and pe_out.stride(2) == 1
    if nope_out is not None:
        assert nope_out.shape == (T, H, 128) and nope_out.dtype == torch.bfloat16 and nope_out.stride(2) == 1
    check(
        load_library().mla_q_rope_bf16(
            _ptr(q), q.stride(0), q.stride(1), T, H, _ptr(positions), _ptr(cos_sin), cos_sin.shape[0],
            int(bool(interleaved)), _ptr(pe_out), pe_out.stride(0), pe_out.stride(1), _ptr(nope_out),
            0 if nope_out is None else nope_out.stride(0), 0 if nope_out is None else nope_out.stride(1),
            _stream(stream),
        ),
        "mla_q_rope_bf16",
    )


def qkv_a_rows(qkv, q_rank: int, q_norm_weight, kv_norm_weight, positions, cos_sin, eps: float, interleaved: bool,
               out=None, stream=None):
    """``qkv [T, q_rank + 576]`` (the fused q_a / kv_a output): RMSNorm of ``qkv[:, :q_rank]`` in place,
    and the latent rows ``[T, 576]`` of ``qkv[:, q_rank:]`` (as ``latent_rows``), in one launch."""
    import torch

    assert qkv.dim() == 2 and qkv.shape[1] == q_rank + 576 and qkv.dtype == torch.bfloat16 and qkv.stride(1) == 1
    assert qkv.is_cuda and q_rank % 8 == 0
    T = qkv.shape[0]
    assert q_norm_weight.shape == (q_rank,) and q_norm_weight.dtype == torch.bfloat16 and q_norm_weight.is_contiguous()
    assert kv_norm_weight.shape == (512,) and kv_norm_weight.dtype == torch.bfloat16 and kv_norm_weight.is_contiguous()
    assert positions.shape == (T,) and positions.dtype == torch.int32 and positions.is_contiguous()
    assert cos_sin.dim() == 2 and cos_sin.shape[1] == 64 and cos_sin.dtype == torch.float32 and cos_sin.is_contiguous()
    if out is None:
        out = torch.empty((T, 576), dtype=torch.bfloat16, device=qkv.device)
    assert out.shape == (T, 576) and out.dtype == torch.bfloat16 and out.stride(1) == 1
    check(
        load_library().mla_qkv_a_rows_bf16(
            _ptr(qkv), qkv.stride(0), q_rank, _ptr(q_norm_weight), _ptr(kv_norm_weight), _ptr(positions),
            _ptr(cos_sin), cos_sin.shape[0], T, float(eps), int(bool(interleaved)), _ptr(out), out.stride(0),
            _stream(stream),
        ),
        "mla_qkv_a_rows_bf16",
    )
    return out
