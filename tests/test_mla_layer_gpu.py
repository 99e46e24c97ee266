"""The MLA layer through the HIP backend on the GPU against the layer oracle.

A serving sequence (two chunked-prefill steps, decode steps, a prefill continuing after decode,
another decode) runs through ``MLAAttentionLayer`` with bf16 weights, the real MLA pool (latent
rows only, on shuffled pages: prefill decompresses every key from them) and the HIP kernels; every step's output is
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
    ctx.kv_cache = create_kvcache_pool(attn, num_pages, page_size, torch.bfloat16, DEV)
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


def test_mla_layer_page_size_one():
    """The reference's default page size (1): decode on token pages, prefill through 64-token
    scratch pages gathered by the backend."""
    steps = [("prefill", {0: 90, 1: 40}), ("decode", {0: 1, 1: 1}), ("prefill", {1: 70}), ("decode", {0: 1, 1: 1})]
    _run_case(H=16, hidden=1024, q_lora=384, steps=steps, page_size=1, seed=7)


def test_mla_layer_kimi_k2_tp8_shard():
    """Kimi-K2's attention over 8 GPUs: 8 heads per GPU, hidden 7168."""
    steps = [("prefill", {0: 90, 1: 40}), ("decode", {0: 1, 1: 1}), ("decode", {0: 1, 1: 1})]
    _run_case(H=8, hidden=7168, q_lora=1536, steps=steps, seed=2)


def test_mla_layer_deepseek_v3_shape():
    """DeepSeek-V3 attention with data-parallel attention: all 128 heads on one GPU (decode runs
    two 64-head groups), hidden 7168, q_lora 1536."""
    steps = [("prefill", {0: 100, 1: 45}), ("decode", {0: 1, 1: 1}), ("prefill", {1: 30}), ("decode", {0: 1, 1: 1})]
    _run_case(H=128, hidden=7168, q_lora=1536, steps=steps, seed=4)


def test_mla_layer_with_page_allocator():
    """Pages allocated step by step by the token-table writer (as the scheduler does), a finished
    request's pages freed and reused by a new request, so rows hold non-contiguous pages."""
    from minisgl_amd.kvcache import PagedTokenTable

    reset_global_ctx()
    gen = torch.Generator().manual_seed(6)
    H, hidden, ps = 16, 1024, 64
    attn = MLAConfig(num_heads=H, num_layers=1, softmax_mscale=softmax_mscale(KIMI_YARN))
    cfg = MLALayerConfig(attn=attn, hidden_size=hidden, q_lora_rank=384, rope_theta=50000.0, max_position=16384,
                         rope_scaling=KIMI_YARN)
    weights = MLAWeights.random(cfg, gen, DEV)
    steps = [("prefill", {0: 150, 1: 90}), ("decode", {0: 1, 1: 1}), ("free", {1: 0}),
             ("prefill", {2: 300}), ("decode", {0: 1, 2: 1}), ("prefill", {0: 70}), ("decode", {0: 1, 2: 1})]
    lens = S.total_lens(steps)
    num_pages = 12
    ctx = Context(page_size=ps)
    set_global_ctx(ctx)
    ctx.page_table = torch.zeros((4, 512), dtype=torch.int32, device=DEV)
    alloc = PagedTokenTable(num_pages, ps, ctx.page_table)
    alloc.free_slots = alloc.free_slots[torch.randperm(num_pages, generator=gen).to(DEV)]  # a long-running server's order
    ctx.kv_cache = create_kvcache_pool(attn, num_pages, ps, torch.bfloat16, DEV)
    backend = create_attention_backend("mla", attn)
    ctx.attn_backend = backend
    layer = MLAAttentionLayer(0, cfg, weights)
    x_hist = {r: torch.randn((L, hidden), generator=gen).to(torch.bfloat16) for r, L in lens.items()}
    Wd = {k: getattr(weights, k).cpu().double() for k in WEIGHT_NAMES}
    kw = dict(num_heads=H, rope_dim=64, rope_theta=50000.0, rope_scaling=dict(KIMI_YARN), interleaved=True,
              scale=attn.softmax_scale, round_bf16=True)
    try:
        for phase, new, after, out in S.run(layer, ctx, backend, x_hist, steps, None, DEV, alloc=alloc):
            torch.cuda.synchronize()
            want = S.expected({r: x.double() for r, x in x_hist.items()}, new, after, Wd, **kw)
            rel = float((out.double().cpu() - want).norm() / want.norm())
            print(f"[mla layer alloc] {phase} {new}: rel err {rel:.2e}, free pages {alloc.free_pages}", flush=True)
            torch.testing.assert_close(out.double().cpu(), want, atol=2e-2, rtol=2e-2)
            assert rel < 1e-2
    finally:
        reset_global_ctx()


def test_mla_layer_decode_graph_replay():
    """A decode layer step captured in a HIP graph and replayed (with eager work between replays)
    gives the eager step's output every time."""
    reset_global_ctx()
    gen = torch.Generator().manual_seed(3)
    H, hidden = 64, 1024
    attn = MLAConfig(num_heads=H, num_layers=1, softmax_mscale=softmax_mscale(KIMI_YARN))
    cfg = MLALayerConfig(attn=attn, hidden_size=hidden, q_lora_rank=384, rope_theta=50000.0, max_position=16384,
                         rope_scaling=KIMI_YARN)
    weights = MLAWeights.random(cfg, gen, DEV)
    steps = [("prefill", {0: 300, 1: 70, 2: 129}), ("decode", {0: 1, 1: 1, 2: 1})]
    lens = S.total_lens(steps)
    tt, num_pages = S.token_table(lens, 64, gen)
    ctx = Context(page_size=64)
    set_global_ctx(ctx)
    ctx.page_table = tt.to(DEV)
    ctx.kv_cache = create_kvcache_pool(attn, num_pages, 64, torch.bfloat16, DEV)
    backend = create_attention_backend("mla", attn)
    ctx.attn_backend = backend
    layer = MLAAttentionLayer(0, cfg, weights)
    x_hist = {r: torch.randn((L, hidden), generator=gen).to(torch.bfloat16) for r, L in lens.items()}
    try:
        outs = [out for *_, out in S.run(layer, ctx, backend, x_hist, steps, tt, DEV)]
        eager = outs[-1].clone()
        # the same decode step again, as a graph: batch tensors are the static inputs
        from minisgl_amd.core import Batch, Req

        reqs = [Req(table_idx=r, cached_len=lens[r] - 1, device_len=lens[r]) for r in sorted(lens)]
        batch = Batch(reqs=reqs, phase="decode")
        batch.padded_reqs = reqs
        batch.positions = torch.tensor([lens[r] - 1 for r in sorted(lens)], dtype=torch.int32, device=DEV)
        batch.out_loc = torch.stack([tt[r, lens[r] - 1] for r in sorted(lens)]).to(DEV)
        x = torch.stack([x_hist[r][lens[r] - 1] for r in sorted(lens)]).to(DEV)
        backend.prepare_metadata(batch)
        stream = torch.cuda.Stream()
        with ctx.forward_batch(batch), torch.cuda.stream(stream):
            layer.forward(x)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                static_out = layer.forward(x)
        torch.cuda.synchronize()
        for i in range(3):
            g.replay()
            torch.cuda.synchronize()
            print(f"[mla layer graph] replay {i}: max diff {float((static_out - eager).abs().max()):.3e}", flush=True)
            torch.testing.assert_close(static_out.float(), eager.float(), atol=1e-2, rtol=1e-2)
            _ = (x.float() * 2).sum().item()  # eager work between replays
    finally:
        reset_global_ctx()
