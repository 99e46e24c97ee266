"""Whole MLA layer steps at the Kimi-K2 shape, for the benchmark.

One step is ``MLAAttentionLayer.forward`` over one batch (projections, RoPE, absorption, the HIP
attention kernels, o_proj) through the real context, pool and backend. Two layers with their own
weights and KV alternate, so that neither a layer's weights (202 MB) nor its KV stays in the
256 MB Infinity Cache between its steps, as in a 61-layer model.

Decode: B=64, lengths U[1024, 8192] (the headline attention batch: same seed, same lengths),
one new token per request. Prefill: B=4 chunks of 2048 tokens on prefixes U[0, 8192] (the prefill
attention batch), every key (prefix and chunk) decompressed from the latent pool by the backend.
Both phases run over a latent-only pool.
"""

from __future__ import annotations

from typing import Dict, List, Sequence

import torch

from ..attention import create_attention_backend
from ..config import MLAConfig
from ..core import Batch, Context, Req, reset_global_ctx, set_global_ctx
from ..kvcache import create_kvcache_pool
from ..layers import MLAAttentionLayer, MLALayerConfig, MLAWeights, softmax_mscale
from .inputs import _lens

KIMI_K2_YARN = (
    ("rope_type", "yarn"),
    ("factor", 32.0),
    ("original_max_position_embeddings", 4096),
    ("beta_fast", 1.0),
    ("beta_slow", 1.0),
    ("mscale", 1.0),
    ("mscale_all_dim", 1.0),
)
HIDDEN, Q_LORA, HEADS, PAGE = 7168, 1536, 64, 64


def kimi_k2_layer_config(num_layers: int) -> MLALayerConfig:
    attn = MLAConfig(num_heads=HEADS, num_layers=num_layers, softmax_mscale=softmax_mscale(KIMI_K2_YARN))
    return MLALayerConfig(attn=attn, hidden_size=HIDDEN, q_lora_rank=Q_LORA, rope_theta=50000.0,
                          max_position=32768, rope_scaling=KIMI_K2_YARN)


def gemm_flops_per_token(cfg: MLALayerConfig, decode: bool) -> int:
    """Projection FLOPs of one new token: q_a, q_b, kv_a, o, plus the absorption (decode)."""
    a = cfg.attn
    H, r = a.num_heads, a.kv_lora_rank
    f = cfg.hidden_size * cfg.q_lora_rank + cfg.q_lora_rank * H * a.qk_head_dim + cfg.hidden_size * a.kv_dim
    f += H * a.v_head_dim * cfg.hidden_size
    if decode:
        f += H * (a.qk_nope_head_dim * r + r * a.v_head_dim)
    return 2 * f


def decompress_flops_per_key(cfg: MLALayerConfig) -> int:
    """Prefill: the per-head K/V decompression of one key, [k_nope | v] = c W_kvb^T."""
    a = cfg.attn
    return 2 * a.kv_lora_rank * a.num_heads * (a.qk_nope_head_dim + a.v_head_dim)


def weight_bytes(w: MLAWeights) -> int:
    return sum(t.numel() * t.element_size() for t in (w.q_a, w.q_a_norm, w.q_b, w.kv_a, w.kv_a_norm, w.kv_b, w.o))


class LayerBench:
    """Context, pool, backend, two layers and one batch; ``step(i)`` runs layer ``i % 2``."""

    def __init__(self, phase: str, lens: Sequence[int], extends: Sequence[int], dev: torch.device, seed: int = 0):
        reset_global_ctx()
        self.cfg = kimi_k2_layer_config(2)
        self.phase = phase
        gen = torch.Generator().manual_seed(seed)
        need = [-(-L // PAGE) for L in lens]
        num_pages = sum(need) + 1
        width = -(-max(need) * PAGE // 32) * 32
        tt = torch.zeros((len(lens) + 1, width), dtype=torch.int32)
        perm = torch.randperm(num_pages, generator=gen)
        off = 0
        for b, n in enumerate(need):
            tt[b, : n * PAGE] = (perm[off : off + n, None] * PAGE + torch.arange(PAGE)).flatten().to(torch.int32)
            off += n
        self.ctx = Context(page_size=PAGE)
        set_global_ctx(self.ctx)
        self.ctx.page_table = tt.to(dev)
        pool = create_kvcache_pool(self.cfg.attn, num_pages, PAGE, torch.bfloat16, dev)
        self.ctx.kv_cache = pool
        gd = torch.Generator(device=dev).manual_seed(seed + 2)
        for c in [pool.latent_cache(i) for i in range(2)]:
            c.copy_(torch.randn(c.shape, generator=gd, device=dev).to(torch.bfloat16))
        self.backend = create_attention_backend("mla", self.cfg.attn)
        self.ctx.attn_backend = self.backend
        self.layers = [MLAAttentionLayer(i, self.cfg, MLAWeights.random(self.cfg, gen, dev)) for i in range(2)]

        reqs = [Req(table_idx=b, cached_len=L - E, device_len=L) for b, (L, E) in enumerate(zip(lens, extends))]
        self.batch = Batch(reqs=reqs, phase=phase)
        self.batch.padded_reqs = reqs
        self.batch.positions = torch.cat([torch.arange(r.cached_len, r.device_len) for r in reqs]).to(torch.int32).to(dev)
        self.batch.out_loc = torch.cat([tt[r.table_idx, r.cached_len : r.device_len] for r in reqs]).to(dev)
        self.backend.prepare_metadata(self.batch)
        self.tokens = sum(extends)
        self.x = torch.randn((self.tokens, HIDDEN), generator=gd, device=dev).to(torch.bfloat16)
        self.lens, self.extends = list(lens), list(extends)

    def step(self, i: int) -> torch.Tensor:
        with self.ctx.forward_batch(self.batch):
            return self.layers[i % 2].forward(self.x)

    def capture(self, stream: torch.cuda.Stream) -> List[torch.cuda.CUDAGraph]:
        """One HIP graph per layer of this batch's step (the serving engine replays decode steps
        from graphs); the batch's metadata tensors are the graphs' static inputs."""
        graphs = []
        with torch.cuda.stream(stream):
            for i in range(2):
                self.step(i)
            torch.cuda.synchronize()
            for i in range(2):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=stream):
                    self.step(i)
                graphs.append(g)
        torch.cuda.synchronize()
        return graphs

    def close(self) -> None:
        reset_global_ctx()


def decode_lens(batch: int = 64, seed: int = 0) -> List[int]:
    """The headline decode batch's lengths (same generator draw as ``make_decode_case``)."""
    return _lens(batch, 1024, 8192, torch.Generator().manual_seed(seed))


def summary(b: LayerBench, ms: float, attn_flops: int, attn_bytes: int) -> Dict[str, float]:
    """Layer-step figures: time, tokens/s, projection + attention FLOPs and HBM bytes."""
    decode = b.phase == "decode"
    gemm = gemm_flops_per_token(b.cfg, decode) * b.tokens
    if not decode:  # every key of every request is decompressed once per layer
        gemm += decompress_flops_per_key(b.cfg) * sum(b.lens)
    w_bytes = weight_bytes(b.layers[0].w)
    act_bytes = b.tokens * HIDDEN * 2 * 2  # x in, out
    flops = gemm + attn_flops
    return {
        "us_per_layer": round(ms * 1e3, 1),
        "tokens_per_s": round(b.tokens / (ms * 1e-3), 1),
        "gemm_gflop": round(gemm / 1e9, 2),
        "attention_gflop": round(attn_flops / 1e9, 2),
        "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
        "weight_mb": round(w_bytes / 1e6, 1),
        "hbm_bytes_min_mb": round((w_bytes + attn_bytes + act_bytes) / 1e6, 1),
        "tb_per_s_min_bytes": round((w_bytes + attn_bytes + act_bytes) / (ms * 1e-3) / 1e12, 3),
    }


class BackendPrefill:
    """The attention backend's prefill path alone over a latent-only pool: store the chunk's latent
    rows, gather every key into scratch pages, decompress with a random ``W_kvb``, prefill kernel.
    ``__call__`` is one layer's ``backend.forward``; two layers alternate."""

    def __init__(self, lens: Sequence[int], extends: Sequence[int], page_size: int, dev: torch.device,
                 seed: int = 0):
        reset_global_ctx()
        attn = MLAConfig(num_heads=HEADS, num_layers=2)
        gen = torch.Generator().manual_seed(seed)
        need = [-(-L // page_size) for L in lens]
        num_pages = sum(need) + 1
        width = -(-max(need) * page_size // 32) * 32
        tt = torch.zeros((len(lens) + 1, width), dtype=torch.int32)
        perm = torch.randperm(num_pages, generator=gen)
        off = 0
        for b, n in enumerate(need):
            tt[b, : n * page_size] = (perm[off : off + n, None] * page_size + torch.arange(page_size)).flatten().to(
                torch.int32)
            off += n
        self.ctx = Context(page_size=page_size)
        set_global_ctx(self.ctx)
        self.ctx.page_table = tt.to(dev)
        pool = create_kvcache_pool(attn, num_pages, page_size, torch.bfloat16, dev)
        self.ctx.kv_cache = pool
        gd = torch.Generator(device=dev).manual_seed(seed + 2)
        for i in range(2):
            c = pool.latent_cache(i)
            c.copy_(torch.randn(c.shape, generator=gd, device=dev).to(torch.bfloat16))
        self.backend = create_attention_backend("mla", attn)
        self.ctx.attn_backend = self.backend
        for i in range(2):
            self.backend.register_kv_b(i, (torch.randn((HEADS * 256, 512), generator=gd, device=dev) / 512 ** 0.5)
                                       .to(torch.bfloat16))
        reqs = [Req(table_idx=b, cached_len=L - E, device_len=L) for b, (L, E) in enumerate(zip(lens, extends))]
        self.batch = Batch(reqs=reqs, phase="prefill")
        self.batch.padded_reqs = reqs
        self.batch.out_loc = torch.cat([tt[r.table_idx, r.cached_len : r.device_len] for r in reqs]).to(dev)
        self.backend.prepare_metadata(self.batch)
        T = sum(extends)
        self.q = torch.randn((T, HEADS, 192), generator=gd, device=dev).to(torch.bfloat16)
        self.k_new = torch.randn((T, 576), generator=gd, device=dev).to(torch.bfloat16)
        self.n = 0

    def __call__(self) -> torch.Tensor:
        with self.ctx.forward_batch(self.batch):
            o = self.backend.forward(self.q, self.k_new, None, self.n % 2, self.batch)
        self.n += 1
        return o

    def close(self) -> None:
        reset_global_ctx()
