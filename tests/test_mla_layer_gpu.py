"""The MLA layer through the HIP backend on the GPU against the layer oracle.

A serving sequence (two chunked-prefill steps, decode steps, a prefill continuing after decode,
another decode) runs through ``MLAAttentionLayer`` with bf16 weights, the real MLA pool (latent
rows + per-head prefill pages on shuffled pages) and the HIP kernels; every step's output is
compared with ``oracle/ref_mla_layer.py`` (decompressed, float64, rounded to bf16 where the
layer keeps bf16 tensors). Tolerance: atol = rtol = 2e-2 elementwise (bf16 outputs), and the
relative Frobenius error of each step below 1e-2.
"""

from __future__ import annotations

import pytest
import torch

from minisgl_amd.attention import create_attention_backend
from minisgl_amd.config import MLAConfig
from minisgl_amd.core import Context, reset_global_ctx, set_global_ctx
from minisgl_amd.kvcache import create_kvcache_pool
from minisgl_amd.layers import MLAAttentionLayer, MLALayerConfig, MLAWeights, softmax_mscale

import mla_layer_scenario as S

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
KIMI_YARN = (
    ("rope_type", "yarn"),
    ("factor", 32.0),
    ("original_max_position_embeddings", 4096),
    ("beta_fast", 1.0),
    ("beta_slow", 1.0),
    ("mscale", 1.0),
    ("mscale_all_dim", 1.0),
)
WEIGHT_NAMES = ("q_a", "q_a_norm", "q_b", "kv_a", "kv_a_norm", "kv_b", "o")


def _run_case(H, hidden, q_lora, steps, page_size=64, seed=0):
    reset_global_ctx()
    gen = torch.Generator().manual_seed(seed)
    attn = MLAConfig(num_heads=H, num_layers=1, softmax_mscale=softmax_mscale(KIMI_YARN))
    cfg = MLALayerConfig(attn=attn, hidden_size=hidden, q_lora_rank=q_lora, rope_theta=50000.0, max_position=16384,
                         rope_scaling=KIMI_YARN)
    weights = MLAWeights.random(cfg, gen, DEV)
    lens = S.total_lens(steps)
    tt, num_pages = S.token_table(lens, page_size, gen)
    print(f"[mla layer] H={H} hidden={hidden} lens={lens} pages={num_pages}", flush=True)
    ctx = Context(page_size=page_size)
    set_global_ctx(ctx)
    ctx.page_table = tt.to(DEV)
    ctx.kv_cache = create_kvcache_pool(attn, num_pages, page_size, torch.bfloat16, DEV, with_prefill_pages=True)
    backend = create_attention_backend("mla", attn)
    ctx.attn_backend = backend
    layer = MLAAttentionLayer(0, cfg, weights)
    x_hist = {r: torch.randn((L, hidden), generator=gen).to(torch.bfloat16) for r, L in lens.items()}
    Wd = {k: getattr(weights, k).cpu().double() for k in WEIGHT_NAMES}
    kw = dict(num_heads=H, rope_dim=64, rope_theta=50000.0, rope_scaling=dict(KIMI_YARN), interleaved=True,
              scale=attn.softmax_scale, round_bf16=True)
    try:
        for phase, new, after, out in S.run(layer, ctx, backend, x_hist, steps, tt, DEV):
            torch.cuda.synchronize()
            want = S.expected({r: x.double() for r, x in x_hist.items()}, new, after, Wd, **kw)
            got = out.double().cpu()
            rel = float((got - want).norm() / want.norm())
            print(f"[mla layer] {phase} {new}: rel err {rel:.2e}", flush=True)
            torch.testing.assert_close(got, want, atol=2e-2, rtol=2e-2, msg=f"{phase} {new}")
            assert rel < 1e-2, f"{phase} {new}: relative error {rel}"
    finally:
        reset_global_ctx()


def test_mla_layer_serving_sequence_16_heads():
    _run_case(H=16, hidden=1024, q_lora=384, steps=S.scaled_steps(5))


def test_mla_layer_kimi_k2_shape():
    """64 heads (Kimi-K2 / DeepSeek-V3 with 1 or 2 way head sharding), hidden 7168, q_lora 1536."""
    steps = [("prefill", {0: 150, 1: 66}), ("decode", {0: 1, 1: 1}), ("prefill", {0: 70}), ("decode", {0: 1, 1: 1})]
    _run_case(H=64, hidden=7168, q_lora=1536, steps=steps, seed=1)
