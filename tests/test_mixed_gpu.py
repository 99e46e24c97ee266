"""A ragged batch sharing radix-prefix pages: decode requests and prefill
chunks whose page-table rows reference the same prefix pages, each half
through its HIP kernel (C ABI) against the CPU oracle.

Tolerances: bf16 output atol = rtol = 2e-2; fp32 natural-log LSE atol 1e-3.
"""

from __future__ import annotations

import pytest
import torch

from minisgl_amd.benchmark.inputs import make_mixed_case
from oracle import ref_mla as R

from test_decode_gpu import run_decode
from test_prefill_gpu import run_prefill

pytestmark = pytest.mark.gpu
DEV = "cuda"
O_TOL = dict(atol=2e-2, rtol=2e-2)
LSE_TOL = dict(atol=1e-3, rtol=0.0)


@pytest.mark.parametrize("groups,ps", [(2, 64), (3, 128)])
def test_mixed_shared_prefix(groups, ps):
    m = make_mixed_case(7, 3, 16, ps, (100, 1500), 200, 2 * ps, groups, seed=groups)
    d, p = m.decode, m.prefill
    # rows of one group start with the same page ids
    assert torch.equal(d.page_table[0, :2], d.page_table[groups, :2])
    o_ref, lse_ref = R.mla_decode(d.q, d.kv_pool, d.page_table, d.lens)
    out, lse, _ = run_decode(d.q.to(DEV), d.kv_pool.to(DEV), d.page_table.to(DEV), d.seq_lens.to(DEV), d.lens, ps, 64)
    torch.testing.assert_close(out, o_ref, **O_TOL)
    torch.testing.assert_close(lse, lse_ref, **LSE_TOL)
    o_ref, lse_ref = R.mla_prefill(p.q, p.k_pool, p.v_pool, p.page_table, p.cu_seqlens_q, p.seq_lens_k)
    out, lse = run_prefill(p)
    torch.testing.assert_close(out, o_ref, **O_TOL)
    torch.testing.assert_close(lse, lse_ref, **LSE_TOL)


def test_mixed_config5_full_size_through_backend():
    """The mixed ragged batch at its full size: 32 decode requests (ctx U[512, 16384]) and 4 prefill
    chunks of 1024 tokens on 2048-token prefixes shared by 8 groups (the page-table rows of a group
    start with the same page ids, as a radix-cache hit gives them, python/minisgl/kvcache/
    radix_cache.py:132-175), 64 heads, page 64. mini-sglang runs a batch as either prefill or decode
    (python/minisgl/core.py:71-97), so the two halves are two batches through one backend's
    prepare_metadata + forward over one latent pool and one token table; each against the oracle
    (prefill: the oracle's decompression of the latent pool, then its chunked prefill)."""
    from minisgl_amd.attention import create_attention_backend
    from minisgl_amd.config import MLAConfig
    from minisgl_amd.core import Batch, Context, Req, reset_global_ctx, set_global_ctx
    from minisgl_amd.kvcache import create_kvcache_pool

    ps, H = 64, 64
    m = make_mixed_case(32, 4, H, ps, (512, 16384), 1024, 2048, 8, device=DEV, seed=0)
    d, p = m.decode, m.prefill
    print(f"[config 5] decode tokens={sum(d.lens)} prefill tokens={sum(p.extends)}", flush=True)
    reset_global_ctx()
    ctx = Context(page_size=ps)
    set_global_ctx(ctx)
    cfg = MLAConfig(num_heads=H, num_layers=1)
    num_pages = d.kv_pool.shape[0]
    pool = create_kvcache_pool(cfg, num_pages, ps, torch.bfloat16, DEV)
    pool.latent_cache(0).copy_(d.kv_pool)
    P = p.k_pool.shape[0]  # the prefill chunks read pages [0, P) only
    ctx.kv_cache = pool
    nd, npf = len(d.lens), len(p.extends)
    width = -(-max(d.page_table.shape[1], p.page_table.shape[1]) * ps // 32) * 32
    tt = torch.zeros((nd + npf + 1, width), dtype=torch.int32, device=DEV)
    for r, pt_row in enumerate(list(d.page_table) + list(p.page_table)):
        toks = (pt_row.long().unsqueeze(1) * ps + torch.arange(ps, device=DEV)).flatten()
        tt[r, : toks.numel()] = toks.to(torch.int32)
    ctx.page_table = tt
    backend = create_attention_backend("mla", cfg)
    ctx.attn_backend = backend

    # decode half: every request decodes its last token (re-storing the row it already holds)
    reqs = [Req(table_idx=b, cached_len=L - 1, device_len=L) for b, L in enumerate(d.lens)]
    batch = Batch(reqs=reqs, phase="decode")
    batch.padded_reqs = reqs
    batch.out_loc = torch.stack([tt[b, L - 1] for b, L in enumerate(d.lens)])
    backend.prepare_metadata(batch)
    k_new = pool.latent_cache(0).view(-1, 576)[batch.out_loc.long()].clone()
    with ctx.forward_batch(batch):
        o = backend.forward(d.q, k_new, None, 0, batch)
    torch.cuda.synchronize()
    o_ref, lse_ref = R.mla_decode(d.q.cpu(), d.kv_pool.cpu(), d.page_table.cpu(), d.lens)
    torch.testing.assert_close(o.float().cpu(), o_ref, **O_TOL)
    torch.testing.assert_close(backend.last_lse.cpu(), lse_ref, **LSE_TOL)
    del o_ref, lse_ref

    # prefill half: each chunk extends its group's 2048-token prefix by 1024 tokens; the keys (the
    # shared prefix and the chunk) are decompressed from the latent pool with the layer's W_kvb
    gen = torch.Generator().manual_seed(3)
    kv_b = (torch.randn((H * 256, 512), generator=gen) / 512 ** 0.5).to(torch.bfloat16).to(DEV)
    backend.register_kv_b(0, kv_b)
    reqs = [Req(table_idx=nd + i, cached_len=P0, device_len=P0 + E)
            for i, (P0, E) in enumerate(zip(p.prefixes, p.extends))]
    batch = Batch(reqs=reqs, phase="prefill")
    batch.padded_reqs = reqs
    batch.out_loc = torch.cat([tt[r.table_idx, r.cached_len : r.device_len] for r in reqs])
    backend.prepare_metadata(batch)
    k_new = pool.latent_cache(0).view(-1, 576)[batch.out_loc.long()].clone()
    with ctx.forward_batch(batch):
        o = backend.forward(p.q, k_new, None, 0, batch)
    torch.cuda.synchronize()
    K, V = R.decompress_pool(pool.latent_cache(0)[:P].cpu(), kv_b.cpu(), H, out_dtype=torch.bfloat16)
    o_ref, lse_ref = R.mla_prefill(p.q.cpu(), K, V, p.page_table.cpu(), p.cu_seqlens_q.cpu(), p.seq_lens_k.cpu())
    torch.testing.assert_close(o.float().cpu(), o_ref, **O_TOL)
    torch.testing.assert_close(backend.last_lse.cpu(), lse_ref, **LSE_TOL)
    reset_global_ctx()
