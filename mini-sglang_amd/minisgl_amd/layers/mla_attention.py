"""DeepSeek-V3 / Kimi-K2 multi-head latent attention layer: the caller of the MLA backend.

The reference's only attention caller is the MHA ``AttentionLayer``
(python/minisgl/layers/attention.py:17-57): split qkv, norm, RoPE, then
``ctx.attn_backend.forward(q, k, v, layer_id, ctx.batch)``. This layer plays the same role for
MLA, with the same context protocol (``get_global_ctx()``: the active batch, the backend, the
KV pool):

* queries: ``q = W_qb . rmsnorm(W_qa . x)`` -> ``[T, H, 192]`` = 128 "nope" + 64 rope dims;
* keys/values: ``[c | k_pe] = W_kva . x`` (``c`` the 512-wide latent, normed; ``k_pe`` the 64
  rope dims shared by all heads); RoPE on ``q_pe`` and ``k_pe`` at ``batch.positions``;
* ``W_kvb`` decompresses the latent per head: ``k_nope = W_UK c`` and ``v = W_UV c``
  (``W_kvb`` rows are ``[H, 128 + 128]`` over the 512 latent columns);
* decode (absorbed): ``q_lat = q_nope W_UK`` -> ``[T, H, 512]``, the backend attends
  ``[q_lat | q_pe]`` over the latent rows ``[c | k_pe]`` and returns ``o_lat [T, H, 512]``,
  then ``o = o_lat W_UV^T`` -> ``[T, H, 128]``;
* prefill (decompressed): the backend stores the chunk's latent rows, decompresses every key of
  each request (prefix and chunk) from the latent pool with this layer's ``W_kvb`` into
  ``k = [k_nope | k_pe]`` and ``v`` per head, and attends ``q`` causally over them;
* ``out = W_o . o``.

The pool holds only latent rows (1152 bytes per token and layer); both phases read them, so a
prefix cached by one request (or by earlier chunks of the same request) serves decode and prefill
alike.

RoPE: the cos/sin cache of python/minisgl/layers/rotary.py:22-31 (``[max_position, d]``, the
``d/2`` cosines then the ``d/2`` sines) with its YaRN frequency blend (rotary.py:92-111);
DeepSeek/Kimi checkpoints rotate interleaved pairs ``(2i, 2i+1)`` (``rope_interleaved``), the
reference's MHA models rotate halves ``(i, i + d/2)``. YaRN also scales the softmax by
``mscale^2`` with ``mscale = 0.1 * mscale_all_dim * ln(factor) + 1`` (the YaRN paper's
attention factor as DeepSeek-V3 applies it), carried by ``MLAConfig.softmax_mscale`` so that
the backend's scale agrees.

The GEMMs are plain library GEMMs (torch.matmul / bmm on hipBLASLt); the elementwise steps
(RMSNorm, the latent row = norm + RoPE, the queries' RoPE and head-major nope copy) and the
attention are the HIP library (``HipLayerOps``, ``minisgl_amd.kernel.lib``). Tensor-parallel
sharding is out of scope (one GPU): ``num_heads`` is this rank's.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Tuple

import torch

from ..config import MLAConfig
from ..core import get_global_ctx
from ..kernel import lib


@dataclass(frozen=True)
class MLALayerConfig:
    attn: MLAConfig
    hidden_size: int = 7168
    q_lora_rank: int = 1536
    rope_theta: float = 50000.0
    max_position: int = 131072
    rms_eps: float = 1e-6
    rope_scaling: Tuple[Tuple[str, Any], ...] | None = None  # e.g. (("rope_type", "yarn"), ("factor", 32.0), ...)
    rope_interleaved: bool = True


def yarn_mscale(factor: float, mscale: float) -> float:
    """YaRN attention factor ``0.1 * mscale * ln(factor) + 1`` (1 for ``factor <= 1``)."""
    return 1.0 if factor <= 1.0 else 0.1 * mscale * math.log(factor) + 1.0


def softmax_mscale(rope_scaling) -> float:
    """The factor whose square multiplies the softmax scale (1 without YaRN)."""
    rs = dict(rope_scaling or ())
    if rs.get("rope_type", rs.get("type")) != "yarn" or not rs.get("mscale_all_dim"):
        return 1.0
    return yarn_mscale(rs["factor"], rs["mscale_all_dim"])


def rope_cos_sin_cache(rotary_dim: int, max_position: int, base: float, rope_scaling=None) -> torch.Tensor:
    """``[max_position, rotary_dim]`` fp32: the cosines of the ``rotary_dim / 2`` frequencies, then the sines."""
    half = rotary_dim // 2
    inv_freq = 1.0 / (base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))
    rs = dict(rope_scaling or ())
    kind = rs.get("rope_type", rs.get("type", "default"))
    amp = 1.0
    if kind == "yarn":
        factor = float(rs["factor"])
        orig = float(rs["original_max_position_embeddings"])

        def dim_of(rotations: float) -> float:  # the dim index whose wavelength fits `rotations` turns in orig
            return rotary_dim * math.log(orig / (rotations * 2 * math.pi)) / (2 * math.log(base))

        lo = max(math.floor(dim_of(rs.get("beta_fast", 32.0))), 0)
        hi = min(math.ceil(dim_of(rs.get("beta_slow", 1.0))), half - 1)
        ramp = ((torch.arange(half, dtype=torch.float32) - lo) / max(hi - lo, 1)).clamp(0.0, 1.0)
        inv_freq = inv_freq * (1.0 - ramp) + (inv_freq / factor) * ramp
        if rs.get("mscale") is not None and rs.get("mscale_all_dim") is not None:
            amp = yarn_mscale(factor, rs["mscale"]) / yarn_mscale(factor, rs["mscale_all_dim"])
    elif kind != "default":
        raise ValueError(f"unsupported rope scaling {kind!r}")
    freqs = torch.arange(max_position, dtype=torch.float32)[:, None] * inv_freq[None, :]
    return torch.cat((freqs.cos() * amp, freqs.sin() * amp), dim=-1)


class HipLayerOps:
    """The layer's elementwise steps on the HIP kernels (bf16 device tensors only; no fallback).

    ``rms_norm(x, w, eps)`` normalises the rows of a fresh projection output in place;
    ``latent_rows(kv, w, positions, cos_sin, eps, interleaved)`` -> ``[T, 576]``;
    ``q_rope(q, positions, cos_sin, interleaved, pe_out, nope_out=None)`` writes the roped rope
    dims to ``pe_out`` (possibly in place) and, if given, the nope dims to ``nope_out``;
    ``qkv_a_rows`` does ``rms_norm`` of the q_a part and ``latent_rows`` of the kv part of the fused
    q_a / kv_a output in one launch."""

    @staticmethod
    def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
        return lib.rmsnorm(x, w, eps, out=x)

    @staticmethod
    def latent_rows(kv, w, positions, cos_sin, eps: float, interleaved: bool) -> torch.Tensor:
        return lib.latent_rows(kv, w, positions, cos_sin, eps, interleaved)

    @staticmethod
    def q_rope(q, positions, cos_sin, interleaved: bool, pe_out, nope_out=None) -> None:
        lib.q_rope(q, positions, cos_sin, interleaved, pe_out, nope_out)

    @staticmethod
    def qkv_a_rows(qkv_a, q_rank: int, q_w, kv_w, positions, cos_sin, eps: float, interleaved: bool):
        """Fused q_a / kv_a output ``[T, q_rank + 576]``: RMSNorm of the q_a part in place and the
        latent rows ``[T, 576]``, one launch. Returns (normed q_a view, latent rows)."""
        latent = lib.qkv_a_rows(qkv_a, q_rank, q_w, kv_w, positions, cos_sin, eps, interleaved)
        return qkv_a[:, :q_rank], latent


@dataclass
class MLAWeights:
    """Weights of one layer, ``[out_features, in_features]`` like torch.nn.Linear."""

    q_a: torch.Tensor  # [q_lora_rank, hidden]
    q_a_norm: torch.Tensor  # [q_lora_rank]
    q_b: torch.Tensor  # [H * 192, q_lora_rank]
    kv_a: torch.Tensor  # [512 + 64, hidden]
    kv_a_norm: torch.Tensor  # [512]
    kv_b: torch.Tensor  # [H * (128 + 128), 512]
    o: torch.Tensor  # [hidden, H * 128]

    @classmethod
    def random(cls, cfg: MLALayerConfig, generator: torch.Generator, device, dtype=torch.bfloat16) -> "MLAWeights":
        """Random-init weights of the layer's shapes (N(0, 1/fan_in); norm weights near 1)."""
        a = cfg.attn
        H = a.num_heads

        def lin(out_f, in_f):
            w = torch.randn((out_f, in_f), generator=generator) / math.sqrt(in_f)
            return w.to(dtype).to(device)

        def norm(n):
            return (1.0 + 0.1 * torch.randn((n,), generator=generator)).to(dtype).to(device)

        return cls(
            q_a=lin(cfg.q_lora_rank, cfg.hidden_size),
            q_a_norm=norm(cfg.q_lora_rank),
            q_b=lin(H * a.qk_head_dim, cfg.q_lora_rank),
            kv_a=lin(a.kv_dim, cfg.hidden_size),
            kv_a_norm=norm(a.kv_lora_rank),
            kv_b=lin(H * (a.qk_nope_head_dim + a.v_head_dim), a.kv_lora_rank),
            o=lin(cfg.hidden_size, H * a.v_head_dim),
        )

    def w_uk(self, cfg: MLAConfig) -> torch.Tensor:
        """``[H, 128, 512]`` view: ``k_nope = W_UK c``."""
        w = self.kv_b.view(cfg.num_heads, cfg.qk_nope_head_dim + cfg.v_head_dim, cfg.kv_lora_rank)
        return w[:, : cfg.qk_nope_head_dim]

    def w_uv(self, cfg: MLAConfig) -> torch.Tensor:
        """``[H, 128, 512]`` view: ``v = W_UV c``."""
        w = self.kv_b.view(cfg.num_heads, cfg.qk_nope_head_dim + cfg.v_head_dim, cfg.kv_lora_rank)
        return w[:, cfg.qk_nope_head_dim :]


class MLAAttentionLayer:
    def __init__(self, layer_id: int, cfg: MLALayerConfig, weights: MLAWeights, ops=None) -> None:
        a = cfg.attn
        assert a.kv_lora_rank == 512 and a.qk_rope_head_dim == 64, "the HIP kernels take 512 + 64 latent rows"
        assert cfg.q_lora_rank % 8 == 0, "the latent part of the fused q_a / kv_a output must stay 16-byte aligned"
        assert abs(a.softmax_mscale - softmax_mscale(cfg.rope_scaling)) < 1e-12, (
            "MLAConfig.softmax_mscale must be softmax_mscale(rope_scaling): the backend's scale comes from it"
        )
        self.layer_id = layer_id
        self.cfg = cfg
        self.w = weights
        self.ops = ops if ops is not None else HipLayerOps()
        device = weights.q_a.device
        self.cos_sin = rope_cos_sin_cache(a.qk_rope_head_dim, cfg.max_position, cfg.rope_theta, cfg.rope_scaling).to(
            device
        )
        # absorption matrices, contiguous per head (batched products take no transposed views)
        # q_a and kv_a read the same input: one GEMM over their stacked rows [q_lora + 576, hidden]
        self.w_qkv_a = torch.cat((weights.q_a, weights.kv_a), dim=0).contiguous()
        self.w_uk = weights.w_uk(a).contiguous()  # [H, 128, 512]
        self.w_uv_t = weights.w_uv(a).transpose(1, 2).contiguous()  # [H, 512, 128]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """``x [T, hidden]`` (the tokens of ``ctx.batch``, in batch order) -> ``[T, hidden]``."""
        a = self.cfg.attn
        ctx = get_global_ctx()
        batch, backend = ctx.batch, ctx.attn_backend
        T, H = x.shape[0], a.num_heads
        ops, eps, inter = self.ops, self.cfg.rms_eps, self.cfg.rope_interleaved
        pos = batch.positions.to(torch.int32)  # no copy when the scheduler already gives int32

        qkv_a = x @ self.w_qkv_a.t()  # [T, q_lora + 576]
        q_a, latent = ops.qkv_a_rows(qkv_a, self.cfg.q_lora_rank, self.w.q_a_norm, self.w.kv_a_norm, pos,
                                     self.cos_sin, eps, inter)  # normed q_a, latent rows [T, 576]
        q = (q_a @ self.w.q_b.t()).view(T, H, a.qk_head_dim)

        if batch.is_decode:
            # absorbed: q_abs = [q_nope W_UK | rope(q_pe)] per head; the nope dims go head-major for the bmm
            q_abs = torch.empty((T, H, a.kv_dim), dtype=x.dtype, device=x.device)
            q_nope_h = torch.empty((H, T, a.qk_nope_head_dim), dtype=x.dtype, device=x.device)
            ops.q_rope(q, pos, self.cos_sin, inter, q_abs[..., a.kv_lora_rank :], q_nope_h.transpose(0, 1))
            # the bmm writes each head's q_nope W_UK straight into the absorbed query's first 512 dims
            torch.bmm(q_nope_h, self.w_uk, out=q_abs[..., : a.kv_lora_rank].transpose(0, 1))
            o_lat = backend.forward(q_abs, latent, None, self.layer_id, batch)  # stores the latent rows
            # o[t, h] = o_lat[t, h] W_UV[h]^T, read and written through head-major views (no copies)
            o = torch.empty((T, H, a.v_head_dim), dtype=x.dtype, device=x.device)
            torch.bmm(o_lat.transpose(0, 1), self.w_uv_t, out=o.transpose(0, 1))
        else:
            ops.q_rope(q, pos, self.cos_sin, inter, q[..., a.qk_nope_head_dim :])  # in place
            # the backend stores the latent rows, then decompresses prefix + chunk with W_kvb
            backend.register_kv_b(self.layer_id, self.w.kv_b)
            o = backend.forward(q, latent, None, self.layer_id, batch)
        return o.reshape(T, H * a.v_head_dim) @ self.w.o.t()
