"""The MLA backend through mini-sglang's interface on the GPU: metadata from a
batch, store + decode per layer, and HIP-graph capture/replay with static
buffers (python/minisgl/engine/graph.py:105-158 drives the same hooks)."""

from __future__ import annotations

import pytest
import torch

from minisgl_amd.attention import create_attention_backend
from minisgl_amd.config import MLAConfig
from minisgl_amd.core import Batch, Context, Req, reset_global_ctx, set_global_ctx
from minisgl_amd.kvcache import create_kvcache_pool
from oracle import ref_mla as R

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
O_TOL = dict(atol=2e-2, rtol=2e-2)
LSE_TOL = dict(atol=1e-3, rtol=0.0)


def _setup(page_size=64, max_req=8, max_seq_len=4096, cached=(100, 1, 640, 3000, 64, 7), seed=0):
    reset_global_ctx()
    ctx = Context(page_size=page_size)
    set_global_ctx(ctx)
    gen = torch.Generator().manual_seed(seed)
    cfg = MLAConfig(num_heads=64, num_layers=2)
    need = [-(-(L + 4) // page_size) for L in cached]  # room for a few decode steps
    num_pages = sum(need) + 8
    pool = create_kvcache_pool(cfg, num_pages + 1, page_size, torch.bfloat16, DEV)  # +1 dummy page
    ctx.kv_cache = pool
    width = -(-max_seq_len // 32) * 32
    tt = torch.zeros((max_req + 1, width), dtype=torch.int32)
    starts = torch.randperm(num_pages, generator=gen)[: sum(need)] * page_size
    off = 0
    for r, n in enumerate(need):  # token table as the reference's CacheManager writes it
        toks = (starts[off : off + n].unsqueeze(1) + torch.arange(page_size)).flatten()
        tt[r, : n * page_size] = toks.to(torch.int32)
        off += n
    tt[max_req].fill_(num_pages * page_size)  # dummy request -> dummy page
    ctx.page_table = tt.to(DEV)
    for layer in range(2):
        pool.latent_cache(layer).copy_(
            torch.randn(pool.latent_cache(layer).shape, generator=gen).to(torch.bfloat16).to(DEV)
        )
    reqs = [Req(table_idx=i, cached_len=L, device_len=L + 1) for i, L in enumerate(cached)]
    backend = create_attention_backend("mla", cfg)
    ctx.attn_backend = backend
    return ctx, cfg, pool, backend, reqs, tt, max_req


def _expected(pool, tt, reqs, q, layer, page_size):
    lens = [r.device_len for r in reqs]
    idx = torch.tensor([r.table_idx for r in reqs], dtype=torch.int32)
    pt = R.page_table_from_tokens(tt, idx, max(lens), page_size)
    return R.mla_decode(q.cpu(), pool.latent_cache(layer).cpu(), pt, lens)


def test_backend_decode_eager():
    ctx, cfg, pool, backend, reqs, tt, _ = _setup()
    gen = torch.Generator().manual_seed(1)
    batch = Batch(reqs=reqs, phase="decode")
    batch.padded_reqs = reqs
    batch.out_loc = torch.tensor([int(tt[r.table_idx, r.device_len - 1]) for r in reqs], dtype=torch.int32, device=DEV)
    backend.prepare_metadata(batch)
    q = torch.randn((len(reqs), 64, 576), generator=gen).to(torch.bfloat16).to(DEV)
    k_new = torch.randn((len(reqs), 576), generator=gen).to(torch.bfloat16).to(DEV)
    with ctx.forward_batch(batch):
        o = backend.forward(q, k_new, k_new[:, :512], 1, batch)
    torch.cuda.synchronize()
    # the new latent rows were stored bit-exactly at out_loc
    flat = pool.latent_cache(1).view(-1, 576)
    assert torch.equal(flat[batch.out_loc.long()].view(torch.int16), k_new.view(torch.int16))
    o_ref, lse_ref = _expected(pool, tt, reqs, q, 1, ctx.page_size)
    torch.testing.assert_close(o.float().cpu(), o_ref, **O_TOL)
    torch.testing.assert_close(backend.last_lse.cpu(), lse_ref, **LSE_TOL)
    md = batch.attn_metadata
    assert torch.equal(md.get_last_indices(len(reqs)).cpu(), torch.arange(len(reqs), dtype=torch.int32))


def _capture_decode(ctx, backend, tt, max_req, bs):
    """Capture one decode forward at batch size ``bs`` (the dummy request fills the batch, as
    python/minisgl/engine/graph.py:130-140 does); returns the graph and its static buffers."""
    dummy = Req(table_idx=max_req, cached_len=0, device_len=1)
    q_static = torch.zeros((bs, 64, 576), dtype=torch.bfloat16, device=DEV)
    k_static = torch.zeros((bs, 576), dtype=torch.bfloat16, device=DEV)
    loc_static = torch.full((bs,), int(tt[max_req, 0]), dtype=torch.int32, device=DEV)
    cap = Batch(reqs=[dummy] * bs, phase="decode")
    cap.padded_reqs = cap.reqs
    cap.out_loc = loc_static
    backend.prepare_for_capture(cap)
    stream = torch.cuda.Stream()
    with ctx.forward_batch(cap), torch.cuda.stream(stream):
        backend.forward(q_static, k_static, None, 0, cap)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            o_static = backend.forward(q_static, k_static, None, 0, cap)
    torch.cuda.synchronize()
    return g, dummy, q_static, k_static, loc_static, o_static


@pytest.mark.parametrize("page_size,graph_max_len", [(64, 4096), (1, 65536)])
def test_backend_decode_graph_replay(page_size, graph_max_len):
    """Capture and replay at page sizes 64 and 1. The captured grid is bounded by the pool's
    tokens, so both run on one CTA per compute unit."""
    print(f"[graph replay] page_size={page_size}", flush=True)
    ctx, cfg, pool, backend, reqs, tt, max_req = _setup(page_size=page_size, seed=2)
    bs = 8
    dummy = Req(table_idx=max_req, cached_len=0, device_len=1)
    backend.init_capture_graph(max_seq_len=graph_max_len, bs_list=[bs])
    assert backend.capture_ctas == backend.num_ctas
    q_static = torch.zeros((bs, 64, 576), dtype=torch.bfloat16, device=DEV)
    k_static = torch.zeros((bs, 576), dtype=torch.bfloat16, device=DEV)
    loc_static = torch.full((bs,), int(tt[max_req, 0]), dtype=torch.int32, device=DEV)
    cap = Batch(reqs=[dummy] * bs, phase="decode")
    cap.padded_reqs = cap.reqs
    cap.out_loc = loc_static
    backend.prepare_for_capture(cap)
    stream = torch.cuda.Stream()
    with ctx.forward_batch(cap), torch.cuda.stream(stream):
        backend.forward(q_static, k_static, None, 0, cap)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            o_static = backend.forward(q_static, k_static, None, 0, cap)
    torch.cuda.synchronize()

    gen = torch.Generator().manual_seed(3)
    for step in range(3):
        live = Batch(reqs=reqs, phase="decode")
        live.padded_reqs = reqs + [dummy] * (bs - len(reqs))
        live.out_loc = torch.tensor(
            [int(tt[r.table_idx, r.device_len - 1]) for r in live.padded_reqs], dtype=torch.int32, device=DEV
        )
        backend.prepare_metadata(live)
        backend.prepare_for_replay(live)
        q = torch.randn((bs, 64, 576), generator=gen).to(torch.bfloat16).to(DEV)
        k_new = torch.randn((bs, 576), generator=gen).to(torch.bfloat16).to(DEV)
        q_static.copy_(q)
        k_static.copy_(k_new)
        loc_static.copy_(live.out_loc)
        g.replay()
        torch.cuda.synchronize()
        n = len(reqs)
        o_ref, lse_ref = _expected(pool, tt, reqs, q[:n], 0, ctx.page_size)
        torch.testing.assert_close(o_static[:n].float().cpu(), o_ref, **O_TOL)
        # eager work between replays, then the requests advance by one token
        _ = (q.float() * 2).sum().item()
        for r in reqs:
            r.complete_one()


@pytest.mark.parametrize("page_size", [64, 32, 16, 1])
def test_backend_prefill_with_prefix(page_size):
    """A prefill batch through the backend: the new per-head K/V rows are stored
    at out_loc, then every request attends its cached prefix and itself causally.
    Pages smaller than 64 tokens (the reference's default page size is 1) go through
    the backend's gather into 64-token scratch pages."""
    print(f"[backend prefill] page_size={page_size}", flush=True)
    reset_global_ctx()
    H = 16
    ctx = Context(page_size=page_size)
    set_global_ctx(ctx)
    gen = torch.Generator().manual_seed(5)
    cfg = MLAConfig(num_heads=H, num_layers=2)
    cached, extends = [0, 130, 64, 700], [300, 1, 77, 129]
    lens = [c + e for c, e in zip(cached, extends)]
    need = [-(-L // page_size) for L in lens]
    num_pages = sum(need) + 3
    pool = create_kvcache_pool(cfg, num_pages, page_size, torch.bfloat16, DEV, with_prefill_pages=True)
    ctx.kv_cache = pool
    tt = torch.zeros((len(lens) + 1, 1024), dtype=torch.int32)
    starts = torch.randperm(num_pages, generator=gen)[: sum(need)] * page_size
    off = 0
    for r, n in enumerate(need):
        tt[r, : n * page_size] = (starts[off : off + n].unsqueeze(1) + torch.arange(page_size)).flatten().to(torch.int32)
        off += n
    ctx.page_table = tt.to(DEV)
    layer = 1
    kc, vc = pool.prefill_k_cache(layer), pool.prefill_v_cache(layer)
    kc.copy_(torch.randn(kc.shape, generator=gen).to(torch.bfloat16).to(DEV))
    vc.copy_(torch.randn(vc.shape, generator=gen).to(torch.bfloat16).to(DEV))
    backend = create_attention_backend("mla", cfg)
    ctx.attn_backend = backend

    reqs = [Req(table_idx=i, cached_len=c, device_len=c + e) for i, (c, e) in enumerate(zip(cached, extends))]
    batch = Batch(reqs=reqs, phase="prefill")
    batch.padded_reqs = reqs
    locs = [int(tt[r.table_idx, t]) for r in reqs for t in range(r.cached_len, r.device_len)]
    batch.out_loc = torch.tensor(locs, dtype=torch.int32, device=DEV)
    backend.prepare_metadata(batch)
    T = sum(extends)
    q = torch.randn((T, H, 192), generator=gen).to(torch.bfloat16).to(DEV)
    k_new = torch.randn((T, H, 192), generator=gen).to(torch.bfloat16).to(DEV)
    v_new = torch.randn((T, H, 128), generator=gen).to(torch.bfloat16).to(DEV)
    with ctx.forward_batch(batch):
        o = backend.forward(q, k_new, v_new, layer, batch)
    torch.cuda.synchronize()
    loc = batch.out_loc.long()
    assert torch.equal(kc.reshape(-1, H, 192)[loc].view(torch.int16), k_new.view(torch.int16))
    assert torch.equal(vc.reshape(-1, H, 128)[loc].view(torch.int16), v_new.view(torch.int16))

    idx = torch.arange(len(reqs), dtype=torch.int32)
    pt = R.page_table_from_tokens(tt, idx, max(lens), page_size)
    cu = torch.tensor([0] + extends, dtype=torch.int32).cumsum(0).to(torch.int32)
    o_ref, lse_ref = R.mla_prefill(q.cpu(), kc.cpu(), vc.cpu(), pt, cu, torch.tensor(lens, dtype=torch.int32))
    assert o.shape == (T, H, 128)
    torch.testing.assert_close(o.float().cpu(), o_ref, **O_TOL)
    torch.testing.assert_close(backend.last_lse.cpu(), lse_ref, **LSE_TOL)
    md = batch.attn_metadata
    assert torch.equal(md.get_last_indices(len(reqs)).cpu(), cu[1:] - 1)


def test_backend_eager_batch_after_capture():
    """A decode batch larger than every captured graph runs eagerly (python/minisgl/engine/
    engine.py:194-196): 200 requests after graphs captured at batch size 8. It plans on its own
    grid and workspace; the graph replayed afterwards still matches the oracle."""
    gen = torch.Generator().manual_seed(11)
    cached = torch.randint(63, 2048, (200,), generator=gen).tolist()
    ctx, cfg, pool, backend, reqs, tt, max_req = _setup(page_size=64, max_req=200, max_seq_len=2112,
                                                        cached=cached, seed=4)
    bs = 8
    backend.init_capture_graph(max_seq_len=2112, bs_list=[bs])
    g, dummy, q_static, k_static, loc_static, o_static = _capture_decode(ctx, backend, tt, max_req, bs)
    graph_ws = backend.ws_graph[0].data_ptr()

    def run_eager():
        batch = Batch(reqs=reqs, phase="decode")
        batch.padded_reqs = reqs
        batch.out_loc = torch.tensor([int(tt[r.table_idx, r.device_len - 1]) for r in reqs], dtype=torch.int32,
                                     device=DEV)
        backend.prepare_metadata(batch)
        assert batch.attn_metadata.workspace[0].data_ptr() != graph_ws
        q = torch.randn((len(reqs), 64, 576), generator=gen).to(torch.bfloat16).to(DEV)
        k_new = pool.latent_cache(0).view(-1, 576)[batch.out_loc.long()].clone()
        with ctx.forward_batch(batch):
            o = backend.forward(q, k_new, None, 0, batch)
        torch.cuda.synchronize()
        print(f"[eager after capture] B={len(reqs)} ctas={batch.attn_metadata.num_ctas} "
              f"slots={batch.attn_metadata.num_slots}", flush=True)
        o_ref, lse_ref = _expected(pool, tt, reqs, q, 0, ctx.page_size)
        torch.testing.assert_close(o.float().cpu(), o_ref, **O_TOL)
        torch.testing.assert_close(backend.last_lse.cpu(), lse_ref, **LSE_TOL)

    run_eager()
    live = Batch(reqs=reqs[:bs], phase="decode")
    live.padded_reqs = reqs[:bs]
    live.out_loc = torch.tensor([int(tt[r.table_idx, r.device_len - 1]) for r in reqs[:bs]], dtype=torch.int32,
                                device=DEV)
    backend.prepare_metadata(live)
    backend.prepare_for_replay(live)
    q = torch.randn((bs, 64, 576), generator=gen).to(torch.bfloat16).to(DEV)
    q_static.copy_(q)
    k_static.copy_(pool.latent_cache(0).view(-1, 576)[live.out_loc.long()])
    loc_static.copy_(live.out_loc)
    g.replay()
    torch.cuda.synchronize()
    o_ref, _ = _expected(pool, tt, reqs[:bs], q, 0, ctx.page_size)
    torch.testing.assert_close(o_static.float().cpu(), o_ref, **O_TOL)
    run_eager()  # and eager again after the replay


def test_backend_decode_page_size_one_kimi_batch():
    """The reference's default page size (1) with the Kimi-K2 batch (B=64, L~U[1024,8192]): one CTA
    per compute unit, whose pieces (up to ~2600 tokens) pass the kernel's 1024-page-id LDS window,
    so the kernel restages page ids mid-piece; output against the oracle."""
    from minisgl_amd.benchmark.inputs import make_decode_case

    reset_global_ctx()
    case = make_decode_case(64, 64, 1, len_range=(1024, 8192), seed=0)
    ctx = Context(page_size=1)
    set_global_ctx(ctx)
    cfg = MLAConfig(num_heads=64, num_layers=1)
    num_pages = case.kv_pool.shape[0]
    pool = create_kvcache_pool(cfg, num_pages, 1, torch.bfloat16, DEV)
    pool.latent_cache(0).copy_(case.kv_pool.to(DEV))
    ctx.kv_cache = pool
    width = -(-case.page_table.shape[1] // 32) * 32
    tt = torch.zeros((65, width), dtype=torch.int32)
    tt[:64, : case.page_table.shape[1]] = case.page_table  # page size 1: token location == page id
    ctx.page_table = tt.to(DEV)
    backend = create_attention_backend("mla", cfg)
    ctx.attn_backend = backend
    reqs = [Req(table_idx=i, cached_len=L - 1, device_len=L) for i, L in enumerate(case.lens)]
    batch = Batch(reqs=reqs, phase="decode")
    batch.padded_reqs = reqs
    batch.out_loc = torch.tensor([int(tt[i, L - 1]) for i, L in enumerate(case.lens)], dtype=torch.int32, device=DEV)
    backend.prepare_metadata(batch)
    assert batch.attn_metadata.num_ctas == backend.num_ctas
    print(f"[backend ps=1] ctas={batch.attn_metadata.num_ctas}", flush=True)
    k_new = pool.latent_cache(0).view(-1, 576)[batch.out_loc.long()].clone()  # re-store the same rows
    with ctx.forward_batch(batch):
        o = backend.forward(case.q.to(DEV), k_new, None, 0, batch)
    torch.cuda.synchronize()
    o_ref, lse_ref = R.mla_decode(case.q, case.kv_pool, case.page_table, case.lens)
    torch.testing.assert_close(o.float().cpu(), o_ref, **O_TOL)
    torch.testing.assert_close(backend.last_lse.cpu(), lse_ref, **LSE_TOL)
    reset_global_ctx()
