"""GPU parity of the chunked MLA prefill kernel (HIP, via the C ABI) against the
CPU oracle: causal over a paged prefix, qk 192, v 128.

Tolerances: bf16 output atol = rtol = 2e-2; fp32 natural-log LSE atol 1e-3.
"""

from __future__ import annotations

import pytest
import torch

from minisgl_amd.benchmark.inputs import make_prefill_case
from minisgl_amd.kernel import lib
from oracle import ref_mla as R

pytestmark = pytest.mark.gpu

DEV = "cuda"
O_TOL = dict(atol=2e-2, rtol=2e-2)
LSE_TOL = dict(atol=1e-3, rtol=0.0)


def run_prefill(case, scale=R.DEFAULT_SCALE):
    T, H, _ = case.q.shape
    out = torch.full((T, H, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse = torch.full((T, H), float("nan"), dtype=torch.float32, device=DEV)
    lib.mla_prefill(
        case.q.to(DEV), case.k_pool.to(DEV), case.v_pool.to(DEV), case.page_table.to(DEV),
        case.cu_seqlens_q.to(DEV), case.seq_lens_k.to(DEV), scale, out, lse,
    )
    torch.cuda.synchronize()
    return out.float().cpu(), lse.cpu()


def check_case(case):
    o_ref, lse_ref = R.mla_prefill(case.q, case.k_pool, case.v_pool, case.page_table, case.cu_seqlens_q,
                                   case.seq_lens_k)
    out, lse = run_prefill(case)
    torch.testing.assert_close(out, o_ref, **O_TOL)
    torch.testing.assert_close(lse, lse_ref, **LSE_TOL)


@pytest.mark.parametrize("ps", [64, 128, 256])
def test_prefill_ragged(ps):
    """Extends that are not multiples of 256 (or 32), prefixes that split pages."""
    case = make_prefill_case(8, ps, extends=[1, 37, 256, 300], prefixes=[0, 95, 64, 513], seed=ps)
    check_case(case)


@pytest.mark.parametrize("heads", [1, 3, 5, 16, 64])
def test_prefill_heads(heads):
    """Head counts 1..64, odd ones included (one head per CTA at these sizes)."""
    case = make_prefill_case(heads, 64, extends=[129, 64], prefixes=[200, 0], seed=heads)
    check_case(case)


def test_prefill_output_rows_8_byte_aligned():
    """An output whose head stride is a multiple of 4 but not 8 elements takes the 8-byte stores:
    the same bits as a contiguous output, and the columns past 128 untouched."""
    case = make_prefill_case(5, 64, extends=[300, 45], prefixes=[77, 640], seed=11)
    T, H, _ = case.q.shape
    out_c, lse_c = run_prefill(case)
    buf = torch.full((T, H, 132), float("nan"), dtype=torch.bfloat16, device=DEV)
    out = buf[..., :128]
    lse = torch.full((T, H), float("nan"), dtype=torch.float32, device=DEV)
    lib.mla_prefill(
        case.q.to(DEV), case.k_pool.to(DEV), case.v_pool.to(DEV), case.page_table.to(DEV),
        case.cu_seqlens_q.to(DEV), case.seq_lens_k.to(DEV), R.DEFAULT_SCALE, out, lse,
    )
    torch.cuda.synchronize()
    assert torch.equal(out.float().cpu(), out_c)
    assert torch.equal(lse.cpu(), lse_c)
    assert torch.isnan(buf[..., 128:].float()).all()


def test_prefill_no_prefix_is_causal_sdpa():
    """Without a prefix the kernel equals plain causal attention (one request)."""
    case = make_prefill_case(4, 64, extends=[300], prefixes=[0], seed=7)
    out, lse = run_prefill(case)
    q = case.q.float().transpose(0, 1)  # [H, E, 192]
    rows = R.token_rows(case.page_table[0], 300, 64)
    k = case.k_pool.reshape(-1, 4, 192)[rows].float().transpose(0, 1)
    v = case.v_pool.reshape(-1, 4, 128)[rows].float().transpose(0, 1)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, scale=R.DEFAULT_SCALE)
    torch.testing.assert_close(out, ref.transpose(0, 1), **O_TOL)


def test_prefill_single_token_extend_is_decode_like():
    """Extend 1 over a long prefix: the last row attends every key."""
    case = make_prefill_case(8, 64, extends=[1, 1], prefixes=[2000, 4095], seed=11)
    check_case(case)


def test_prefill_long_extend_multiple_blocks():
    case = make_prefill_case(4, 64, extends=[1024, 700], prefixes=[1500, 3], seed=12)
    check_case(case)


@pytest.mark.parametrize("heads", [16, 64])
def test_prefill_decompressed_layout_bit_exact(heads):
    """The same K/V values laid out as the latent decompression writes them (per key one row
    [head h: k_nope | v, ..., rope shared by all heads], 64-row pages in another order) give the
    per-head page layout's result bit for bit: only the addressing differs
    (mla_prefill_strided_bf16 vs mla_prefill_bf16)."""
    g = torch.Generator().manual_seed(heads)
    case = make_prefill_case(heads, 64, extends=[300, 1, 77], prefixes=[130, 700, 0], seed=heads)
    rope = torch.randn((case.k_pool.shape[0], 64, 64), generator=g).to(torch.bfloat16)
    case.k_pool[..., 128:] = rope[:, :, None, :]  # one rope row per token, as MLA's k_pe
    out_a, lse_a = run_prefill(case)
    P = case.k_pool.shape[0]
    perm = torch.randperm(P, generator=g)  # scratch page of pool page p: perm[p]
    rows = torch.zeros((P, 64, heads * 256 + 64), dtype=torch.bfloat16)
    rows_h = rows[..., : heads * 256].view(P, 64, heads, 256)
    rows_h[perm, :, :, :128] = case.k_pool[..., :128]
    rows_h[perm, :, :, 128:] = case.v_pool
    rows[perm, :, heads * 256 :] = rope
    pt = perm[case.page_table.long()].to(torch.int32)
    T = case.q.shape[0]
    out = torch.full((T, heads, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse = torch.full((T, heads), float("nan"), dtype=torch.float32, device=DEV)
    lib.mla_prefill_decompressed(case.q.to(DEV), rows.view(P * 64, -1).to(DEV), pt.to(DEV),
                                 case.cu_seqlens_q.to(DEV), case.seq_lens_k.to(DEV), T, R.DEFAULT_SCALE, out, lse)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu().view(torch.int16), out_a.to(torch.bfloat16).view(torch.int16))
    assert torch.equal(lse.cpu(), lse_a)


def test_prefill_small_pages_rejected():
    case = make_prefill_case(2, 32, extends=[10], prefixes=[5], seed=1)
    with pytest.raises(lib.MLAKernelError, match="page_size"):
        run_prefill(case)


def test_prefill_growing_logits_rescale():
    """Scores that grow along the keys force the running max to move many times."""
    case = make_prefill_case(2, 64, extends=[300], prefixes=[700], seed=13)
    ramp = torch.linspace(0, 40, case.k_pool.shape[0] * 64).view(-1, 64, 1)
    k = case.k_pool.float()
    k[..., 0] = ramp  # dim 0 of every head grows with the flat row index
    case.k_pool = k.to(torch.bfloat16)
    case.q[..., 0] = 8.0
    check_case(case)


def test_prefill_prefix_beyond_staged_page_ids():
    """More pages than the kernel stages in LDS (1024 at page size 64): the page ids are read from
    the table per stage."""
    case = make_prefill_case(2, 64, extends=[40, 300], prefixes=[66000, 65500], seed=14)
    check_case(case)


def _set_key_dim0(case, fn):
    """k[..., 0] of every head := fn(logical token index, request length), in each request's order."""
    k = case.k_pool.float()
    ps = case.page_size
    for b, L in enumerate(case.seq_lens_k.tolist()):
        rows = R.token_rows(case.page_table[b].cpu(), L, ps)
        t = torch.arange(L, dtype=torch.float32)
        k.view(-1, *k.shape[2:])[rows, :, 0] = fn(t, L).unsqueeze(1)
    case.k_pool = k.to(torch.bfloat16)


def test_prefill_reference_moves_along_keys():
    """Scores that climb ~50 (log2 units) along the keys: the row reference has to move."""
    case = make_prefill_case(2, 64, extends=[300, 77], prefixes=[1500, 400], seed=15)
    _set_key_dim0(case, lambda t, L: 60.0 * t / L)
    case.q[..., 0] = 8.0
    check_case(case)


def test_prefill_single_dominant_key():
    """One key scores ~200 above the rest, in the middle of the prefix."""
    case = make_prefill_case(4, 64, extends=[200], prefixes=[900], seed=16)
    _set_key_dim0(case, lambda t, L: torch.where(t == 517, 240.0, 0.0))
    case.q[..., 0] = 8.0
    check_case(case)


def test_prefill_full_bench_batch_sampled_rows_and_chunking():
    """The benchmark's batch at full size (B=4, H=64, E=2048, P~U[0,8192], page 64): sampled query
    rows of every request against the oracle, and chunk invariance: the same requests prefilled as
    two 1024-row chunks (the first over keys up to P + 1024, the second over the whole prefix)
    give the full run's rows bit for bit."""
    g = torch.Generator().manual_seed(0)
    prefixes = torch.randint(0, 8193, (4,), generator=g).tolist()
    print(f"[prefill full] prefixes={prefixes}", flush=True)
    E, H, ps = 2048, 64, 64
    case = make_prefill_case(H, ps, extends=[E] * 4, prefixes=prefixes, device=DEV, seed=0)
    T = 4 * E

    def run(q, cu, lens):
        out = torch.full((q.shape[0], H, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
        lse = torch.full((q.shape[0], H), float("nan"), dtype=torch.float32, device=DEV)
        lib.mla_prefill(q, case.k_pool, case.v_pool, case.page_table, cu, lens, R.DEFAULT_SCALE, out, lse)
        torch.cuda.synchronize()
        return out, lse

    out, lse = run(case.q, case.cu_seqlens_q, case.seq_lens_k)
    # chunk invariance
    half = E // 2
    cu_half = torch.arange(0, T // 2 + 1, half, dtype=torch.int32, device=DEV)
    first = torch.cat([torch.arange(b * E, b * E + half) for b in range(4)]).to(DEV)
    second = first + half
    lens_first = torch.tensor([P + half for P in prefixes], dtype=torch.int32, device=DEV)
    o1, l1 = run(case.q[first].contiguous(), cu_half, lens_first)
    o2, l2 = run(case.q[second].contiguous(), cu_half, case.seq_lens_k)
    assert torch.equal(o1.view(torch.int16), out[first].view(torch.int16)) and torch.equal(l1, lse[first])
    assert torch.equal(o2.view(torch.int16), out[second].view(torch.int16)) and torch.equal(l2, lse[second])
    # sampled rows against the oracle: block edges, the diagonal's ends, and random rows
    kflat = case.k_pool.reshape(-1, H, 192)
    vflat = case.v_pool.reshape(-1, H, 128)
    gen = torch.Generator().manual_seed(1)
    for b, P in enumerate(prefixes):
        L = P + E
        rows = R.token_rows(case.page_table[b].cpu(), L, ps).to(DEV)
        k = kflat[rows].float().cpu().transpose(0, 1)
        v = vflat[rows].float().cpu().transpose(0, 1)
        pick = torch.cat((torch.tensor([0, 1, 31, 32, 255, 256, 1023, 1024, E - 2, E - 1]),
                          torch.randint(0, E, (22,), generator=gen))).unique()
        qs = case.q[b * E + pick.to(DEV)].float().cpu().transpose(0, 1)
        mask = torch.arange(L)[None, :] <= (P + pick)[:, None]
        o_ref, lse_ref = R._attend(qs, k, v, R.DEFAULT_SCALE, mask[None])
        torch.testing.assert_close(out[b * E + pick.to(DEV)].float().cpu(), o_ref.transpose(0, 1), **O_TOL)
        torch.testing.assert_close(lse[b * E + pick.to(DEV)].cpu(), lse_ref.transpose(0, 1), **LSE_TOL)


def test_prefill_head_pairs_odd_heads_chunk_invariant():
    """A batch large enough for two heads per CTA (one 8192-row extend: 33 row blocks x 63 heads
    is at least 8 CTAs per compute unit) with an odd head count, so the last CTA of each block
    runs one head: bit for bit the same as the same rows prefilled as 1024-row chunks, which are
    small enough to run one head per CTA."""
    H, E, P, ps = 63, 8192, 300, 64
    print(f"[prefill head pairs] H={H} E={E} P={P}", flush=True)
    case = make_prefill_case(H, ps, extends=[E], prefixes=[P], device=DEV, seed=5)

    def run(q, cu, lens):
        out = torch.full((q.shape[0], H, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
        lse = torch.full((q.shape[0], H), float("nan"), dtype=torch.float32, device=DEV)
        lib.mla_prefill(q, case.k_pool, case.v_pool, case.page_table, cu, lens, R.DEFAULT_SCALE, out, lse)
        torch.cuda.synchronize()
        return out, lse

    out, lse = run(case.q, case.cu_seqlens_q, case.seq_lens_k)
    assert not torch.isnan(lse).any()
    C = 1024
    cu = torch.tensor([0, C], dtype=torch.int32, device=DEV)
    for c in range(E // C):
        lens = torch.tensor([P + C * (c + 1)], dtype=torch.int32, device=DEV)
        o, l = run(case.q[C * c: C * (c + 1)].contiguous(), cu, lens)
        assert torch.equal(o.view(torch.int16), out[C * c: C * (c + 1)].view(torch.int16)), c
        assert torch.equal(l, lse[C * c: C * (c + 1)]), c


def test_prefill_head_pairs_unstaged_long_prefix_chunk_invariant():
    """Two heads per CTA over more stages than the kernel stages sources for (a 30,000-token
    prefix: the later query blocks read their page ids per stage, so the second head's sources
    are computed, not moved): bit for bit the same as 1024-row chunks (one head per CTA)."""
    H, E, P, ps = 64, 8192, 30000, 64
    print(f"[prefill head pairs, long prefix] H={H} E={E} P={P}", flush=True)
    case = make_prefill_case(H, ps, extends=[E], prefixes=[P], device=DEV, seed=6)

    def run(q, cu, lens):
        out = torch.full((q.shape[0], H, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
        lse = torch.full((q.shape[0], H), float("nan"), dtype=torch.float32, device=DEV)
        lib.mla_prefill(q, case.k_pool, case.v_pool, case.page_table, cu, lens, R.DEFAULT_SCALE, out, lse)
        torch.cuda.synchronize()
        return out, lse

    out, lse = run(case.q, case.cu_seqlens_q, case.seq_lens_k)
    assert not torch.isnan(lse).any()
    C = 1024
    cu = torch.tensor([0, C], dtype=torch.int32, device=DEV)
    for c in range(E // C):
        lens = torch.tensor([P + C * (c + 1)], dtype=torch.int32, device=DEV)
        o, l = run(case.q[C * c: C * (c + 1)].contiguous(), cu, lens)
        assert torch.equal(o.view(torch.int16), out[C * c: C * (c + 1)].view(torch.int16)), c
        assert torch.equal(l, lse[C * c: C * (c + 1)]), c


def test_prefill_full_bench_request_every_row():
    """Two requests of the benchmark's batch at full size (H=64, E=2048, page 64, the batch's
    smallest and largest prefixes), every one of their 2048 x 64 output rows and LSEs against the
    oracle (not sampled). The whole four-request batch runs in one launch, as in the benchmark."""
    g = torch.Generator().manual_seed(0)
    prefixes = torch.randint(0, 8193, (4,), generator=g).tolist()
    E, H, ps = 2048, 64, 64
    case = make_prefill_case(H, ps, extends=[E] * 4, prefixes=prefixes, device=DEV, seed=0)
    T = 4 * E
    out = torch.full((T, H, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse = torch.full((T, H), float("nan"), dtype=torch.float32, device=DEV)
    lib.mla_prefill(case.q, case.k_pool, case.v_pool, case.page_table, case.cu_seqlens_q, case.seq_lens_k,
                    R.DEFAULT_SCALE, out, lse)
    torch.cuda.synchronize()
    kflat = case.k_pool.reshape(-1, H, 192)
    vflat = case.v_pool.reshape(-1, H, 128)
    for b in (min(range(4), key=lambda i: prefixes[i]), max(range(4), key=lambda i: prefixes[i])):
        P = prefixes[b]
        L = P + E
        print(f"[prefill every row] request {b} prefix {P}", flush=True)
        rows = R.token_rows(case.page_table[b].cpu(), L, ps).to(DEV)
        k = kflat[rows].float().cpu().transpose(0, 1)
        v = vflat[rows].float().cpu().transpose(0, 1)
        qb = case.q[b * E : (b + 1) * E].float().cpu().transpose(0, 1)
        mask = (torch.arange(L)[None, :] <= (P + torch.arange(E))[:, None])[None]
        got_o = out[b * E : (b + 1) * E].float().cpu()
        got_l = lse[b * E : (b + 1) * E].cpu()
        for h0 in range(0, H, 16):  # the oracle's math in head chunks (bounded host memory)
            o_ref, lse_ref = R._attend(qb[h0 : h0 + 16], k[h0 : h0 + 16], v[h0 : h0 + 16], R.DEFAULT_SCALE, mask)
            torch.testing.assert_close(got_o[:, h0 : h0 + 16], o_ref.transpose(0, 1), **O_TOL)
            torch.testing.assert_close(got_l[:, h0 : h0 + 16], lse_ref.transpose(0, 1), **LSE_TOL)


def test_prefill_many_requests():
    """130 requests in one launch (more than one 64-request chunk of the kernel's work-item scan):
    extends 1..300 on ragged prefixes 0..900, empty-prefix and one-token requests among them."""
    g = torch.Generator().manual_seed(12)
    n = 130
    extends = torch.randint(1, 301, (n,), generator=g).tolist()
    prefixes = torch.randint(0, 901, (n,), generator=g).tolist()
    extends[:4] = [1, 1, 300, 32]
    prefixes[:4] = [0, 700, 0, 64]
    case = make_prefill_case(8, 64, extends=extends, prefixes=prefixes, seed=12)
    check_case(case)
