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


def _prefill_setup(page_size, cached, extends, H=16, seed=5, scratch_rows=None):
    """Context, latent pool (random rows on 2 layers), token table and backend for a prefill batch."""
    reset_global_ctx()
    ctx = Context(page_size=page_size)
    set_global_ctx(ctx)
    gen = torch.Generator().manual_seed(seed)
    cfg = MLAConfig(num_heads=H, num_layers=2)
    lens = [c + e for c, e in zip(cached, extends)]
    need = [-(-L // page_size) for L in lens]
    num_pages = sum(need) + 3
    pool = create_kvcache_pool(cfg, num_pages, page_size, torch.bfloat16, DEV)
    ctx.kv_cache = pool
    width = -(-max(n * page_size for n in need) // 32) * 32
    tt = torch.zeros((len(lens) + 1, width), dtype=torch.int32)
    starts = torch.randperm(num_pages, generator=gen)[: sum(need)] * page_size
    off = 0
    for r, n in enumerate(need):
        tt[r, : n * page_size] = (starts[off : off + n].unsqueeze(1) + torch.arange(page_size)).flatten().to(torch.int32)
        off += n
    ctx.page_table = tt.to(DEV)
    for layer in range(2):
        c = pool.latent_cache(layer)
        c.copy_(torch.randn(c.shape, generator=gen).to(torch.bfloat16).to(DEV))
    if scratch_rows is None:
        backend = create_attention_backend("mla", cfg)
    else:
        from minisgl_amd.attention.mla import MLAAttnBackend

        backend = MLAAttnBackend(cfg, prefill_scratch_rows=scratch_rows)
    ctx.attn_backend = backend
    kv_b = (torch.randn((H * 256, 512), generator=gen) / 512 ** 0.5).to(torch.bfloat16).to(DEV)
    return ctx, pool, backend, tt, lens, kv_b, gen


def _run_prefill(ctx, pool, backend, tt, cached, extends, kv_b, gen, layer=1, H=16):
    """One prefill batch through backend.forward (latent rows of the chunk stored, prefix + chunk
    decompressed with kv_b); returns (o, lse, batch, q) and checks the stored rows bit for bit."""
    backend.register_kv_b(layer, kv_b)
    reqs = [Req(table_idx=i, cached_len=c, device_len=c + e) for i, (c, e) in enumerate(zip(cached, extends))]
    batch = Batch(reqs=reqs, phase="prefill")
    batch.padded_reqs = reqs
    locs = [int(tt[r.table_idx, t]) for r in reqs for t in range(r.cached_len, r.device_len)]
    batch.out_loc = torch.tensor(locs, dtype=torch.int32, device=DEV)
    backend.prepare_metadata(batch)
    T = sum(extends)
    q = torch.randn((T, H, 192), generator=gen).to(torch.bfloat16).to(DEV)
    k_new = torch.randn((T, 576), generator=gen).to(torch.bfloat16).to(DEV)
    with ctx.forward_batch(batch):
        o = backend.forward(q, k_new, None, layer, batch)
    torch.cuda.synchronize()
    stored = pool.latent_cache(layer).reshape(-1, 576)[batch.out_loc.long()]
    assert torch.equal(stored.view(torch.int16), k_new.view(torch.int16))
    return o, backend.last_lse, batch, q


def _prefill_expected(pool, tt, cached, extends, kv_b, q, layer, page_size, H):
    """Oracle: the latent pool decompressed per head (bf16 rows, as the GPU's GEMM writes them), then
    chunked prefill over it."""
    lens = [c + e for c, e in zip(cached, extends)]
    K, V = R.decompress_pool(pool.latent_cache(layer).cpu(), kv_b.cpu(), H, out_dtype=torch.bfloat16)
    idx = torch.arange(len(lens), dtype=torch.int32)
    pt = R.page_table_from_tokens(tt, idx, max(lens), page_size)
    cu = torch.tensor([0] + list(extends), dtype=torch.int32).cumsum(0).to(torch.int32)
    return R.mla_prefill(q.cpu(), K, V, pt, cu, torch.tensor(lens, dtype=torch.int32)), cu


@pytest.mark.parametrize("page_size", [128, 64, 32, 16, 1])
def test_backend_prefill_from_latent_pool(page_size):
    """A prefill batch through the backend over a latent-only pool: the chunk's latent rows are
    stored at out_loc (bit-exact), every key of each request (cached prefix and chunk) is gathered
    into 64-token scratch pages and decompressed per head with the layer's W_kvb, and every request
    attends its prefix and itself causally. Any pool page size (the reference's default is 1)."""
    print(f"[backend prefill] page_size={page_size}", flush=True)
    H = 16
    cached, extends = [0, 130, 64, 700], [300, 1, 77, 129]
    ctx, pool, backend, tt, lens, kv_b, gen = _prefill_setup(page_size, cached, extends, H)
    o, lse, batch, q = _run_prefill(ctx, pool, backend, tt, cached, extends, kv_b, gen, H=H)
    (o_ref, lse_ref), cu = _prefill_expected(pool, tt, cached, extends, kv_b, q, 1, page_size, H)
    T = sum(extends)
    assert o.shape == (T, H, 128)
    torch.testing.assert_close(o.float().cpu(), o_ref, **O_TOL)
    torch.testing.assert_close(lse.cpu(), lse_ref, **LSE_TOL)
    md = batch.attn_metadata
    assert len(md.prefill_plan) == 1
    assert torch.equal(md.get_last_indices(len(lens)).cpu(), cu[1:] - 1)
    reset_global_ctx()


def test_backend_prefill_in_passes():
    """A decompression scratch of 512 rows: the batch runs as several passes of whole requests, one
    request (1300 keys) longer than the scratch, which then grows to hold it."""
    H = 16
    cached, extends = [100, 300, 1200, 0, 40, 64], [28, 100, 100, 200, 1, 63]
    ctx, pool, backend, tt, lens, kv_b, gen = _prefill_setup(64, cached, extends, H, seed=8, scratch_rows=512)
    o, lse, batch, q = _run_prefill(ctx, pool, backend, tt, cached, extends, kv_b, gen, H=H)
    plan = batch.attn_metadata.prefill_plan
    print(f"[prefill passes] {[(p[0], p[1], p[2]) for p in plan]}", flush=True)
    assert len(plan) >= 3 and any(p[2] > 512 for p in plan)
    (o_ref, lse_ref), _ = _prefill_expected(pool, tt, cached, extends, kv_b, q, 1, 64, H)
    torch.testing.assert_close(o.float().cpu(), o_ref, **O_TOL)
    torch.testing.assert_close(lse.cpu(), lse_ref, **LSE_TOL)
    reset_global_ctx()


def test_backend_prefill_many_requests():
    """130 prefill requests in one batch through the backend (extends 1..300 on cached prefixes
    0..900): more requests than one 64-request chunk of the kernel's work-item scan, decompressed
    from the latent pool and checked against the oracle."""
    H = 8
    g = torch.Generator().manual_seed(13)
    n = 130
    extends = torch.randint(1, 301, (n,), generator=g).tolist()
    cached = torch.randint(0, 901, (n,), generator=g).tolist()
    cached[:3], extends[:3] = [0, 500, 0], [1, 1, 300]
    ctx, pool, backend, tt, lens, kv_b, gen = _prefill_setup(64, cached, extends, H, seed=13)
    o, lse, batch, q = _run_prefill(ctx, pool, backend, tt, cached, extends, kv_b, gen, H=H)
    (o_ref, lse_ref), cu = _prefill_expected(pool, tt, cached, extends, kv_b, q, 1, 64, H)
    torch.testing.assert_close(o.float().cpu(), o_ref, **O_TOL)
    torch.testing.assert_close(lse.cpu(), lse_ref, **LSE_TOL)
    assert torch.equal(batch.attn_metadata.get_last_indices(n).cpu(), cu[1:] - 1)
    reset_global_ctx()


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


def test_backend_reserves_the_bytes_it_reports():
    """An engine sizes the pool from the free memory before the backend exists
    (python/minisgl/engine/engine.py:148-165): backend_device_bytes gives the backend's own device
    memory beforehand, and with reserve_scratch the constructor allocates the prefill scratch and
    the eager decode workspace at once, within that figure; a decode and a prefill afterwards
    allocate no further scratch or workspace."""
    from minisgl_amd.attention.mla import (MLAAttnBackend, backend_device_bytes, decode_workspace_bytes,
                                           prefill_scratch_bytes)
    from minisgl_amd.kernel import lib

    cus = lib.device_cu_count(0)
    H, rows, max_req, max_seq_len = 64, 8192, 8, 4096
    reserve = backend_device_bytes(H, cus, max_req, max_seq_len, prefill_scratch_rows=rows)
    ctx, cfg, pool, _, reqs, tt, _ = _setup(max_req=max_req, max_seq_len=max_seq_len)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(DEV)
    backend = MLAAttnBackend(cfg, prefill_scratch_rows=rows, reserve_scratch=True)
    held = torch.cuda.memory_allocated(DEV) - before
    expect = prefill_scratch_bytes(H, rows) + decode_workspace_bytes(H, 2 * cus)
    assert expect <= held <= reserve + 4096, (held, expect, reserve)
    ctx.attn_backend = backend
    ws, scratch = backend.ws_eager[0], backend.scratch_rows
    gen = torch.Generator().manual_seed(3)
    batch = Batch(reqs=reqs, phase="decode")
    batch.padded_reqs = reqs
    batch.out_loc = torch.tensor([int(tt[r.table_idx, r.device_len - 1]) for r in reqs], dtype=torch.int32, device=DEV)
    backend.prepare_metadata(batch)
    q = torch.randn((len(reqs), H, 576), generator=gen).to(torch.bfloat16).to(DEV)
    k_new = torch.randn((len(reqs), 576), generator=gen).to(torch.bfloat16).to(DEV)
    with ctx.forward_batch(batch):
        o = backend.forward(q, k_new, k_new[:, :512], 0, batch)
    torch.cuda.synchronize()
    o_ref, lse_ref = _expected(pool, tt, reqs, q, 0, ctx.page_size)
    torch.testing.assert_close(o.float().cpu(), o_ref, **O_TOL)
    assert backend.ws_eager[0] is ws and backend.scratch_rows is scratch
