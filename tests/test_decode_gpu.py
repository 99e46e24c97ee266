"""GPU parity of the absorbed-MLA decode path (HIP kernels via the C ABI)
against the CPU oracle and the committed golden fixture.

Tolerances: bf16 output atol = rtol = 2e-2; fp32 natural-log LSE atol 1e-3;
store, page-table gather bit-exact.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from minisgl_amd.benchmark.inputs import make_decode_case
from minisgl_amd.kernel import lib
from oracle import ref_mla as R

pytestmark = pytest.mark.gpu

DEV = "cuda"
HERE = os.path.dirname(os.path.abspath(__file__))
O_TOL = dict(atol=2e-2, rtol=2e-2)
LSE_TOL = dict(atol=1e-3, rtol=0.0)


def run_decode(q, kv, pt, seq_lens, lens, ps, num_ctas, scale=R.DEFAULT_SCALE):
    B, H, _ = q.shape
    plan_np, slots = lib.decode_plan(lens, ps, num_ctas)
    plan = torch.from_numpy(plan_np).to(DEV)
    ws_o, ws_lse = lib.decode_workspace(slots, H, DEV)
    out = torch.full((B, H, 512), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse = torch.full((B, H), float("nan"), dtype=torch.float32, device=DEV)
    lib.mla_decode(q, kv, pt, seq_lens, plan, num_ctas, ws_o, ws_lse, scale, out, lse)
    torch.cuda.synchronize()
    return out.float().cpu(), lse.cpu(), slots


def check_case(case, num_ctas):
    o_ref, lse_ref = R.mla_decode(case.q, case.kv_pool, case.page_table, case.lens)
    out, lse, _ = run_decode(
        case.q.to(DEV), case.kv_pool.to(DEV), case.page_table.to(DEV), case.seq_lens.to(DEV), case.lens,
        case.page_size, num_ctas,
    )
    nonempty = torch.tensor([L > 0 for L in case.lens])
    torch.testing.assert_close(out[nonempty], o_ref[nonempty], **O_TOL)
    torch.testing.assert_close(lse[nonempty], lse_ref[nonempty], **LSE_TOL)
    if (~nonempty).any():
        assert torch.all(out[~nonempty] == 0) and torch.all(torch.isneginf(lse[~nonempty]))


@pytest.mark.parametrize("num_ctas", [256, 7])
def test_decode_cpu_reference_shape(num_ctas):
    """B=4, 16 heads, page_size 1, lengths U[64, 512] (the CPU-reference workload)."""
    case = make_decode_case(4, 16, 1, len_range=(64, 512))
    check_case(case, num_ctas)


@pytest.mark.parametrize("num_ctas", [256, 5, 1])
def test_decode_ragged_edges_ps64(num_ctas):
    case = make_decode_case(8, 64, 64, lens=[1, 31, 32, 33, 63, 64, 65, 1000])
    check_case(case, num_ctas)


@pytest.mark.parametrize("heads,ps", [(32, 16), (48, 32), (16, 128), (64, 2)])
def test_decode_heads_and_page_sizes(heads, ps):
    case = make_decode_case(5, heads, ps, len_range=(1, 700), seed=heads + ps)
    check_case(case, 64)


@pytest.mark.parametrize("heads,ps", [(1, 64), (8, 64), (8, 16), (20, 32), (63, 128), (128, 64), (96, 16)])
def test_decode_tensor_parallel_head_counts(heads, ps):
    """Head counts that are not a multiple of 16 (a tensor-parallel shard: Kimi-K2 over 8 GPUs has
    8 heads per GPU): the last wave's lanes without a head compute nothing that is stored. More
    than 64 heads (DeepSeek-V3's 128 with attention data parallelism) run in groups of 64."""
    print(f"[decode heads] heads={heads} ps={ps}", flush=True)
    case = make_decode_case(6, heads, ps, lens=[1, 64, 65, 700, 2048, 33], seed=heads * 7 + ps)
    check_case(case, 64)
    check_case(case, 3)
    # outputs inside a wider buffer: the head slot past `heads` must stay untouched
    B = len(case.lens)
    plan_np, slots = lib.decode_plan(case.lens, ps, 3)
    plan = torch.from_numpy(plan_np).to(DEV)
    ws_o, ws_lse = lib.decode_workspace(slots, heads, DEV)
    wide = torch.full((B, heads + 1, 512), 7.0, dtype=torch.bfloat16, device=DEV)
    wide_lse = torch.full((B, heads + 1), 7.0, dtype=torch.float32, device=DEV)
    lib.mla_decode(case.q.to(DEV), case.kv_pool.to(DEV), case.page_table.to(DEV), case.seq_lens.to(DEV), plan, 3,
                   ws_o, ws_lse, R.DEFAULT_SCALE, wide[:, :heads], wide_lse[:, :heads])
    torch.cuda.synchronize()
    assert torch.all(wide[:, heads] == 7.0) and torch.all(wide_lse[:, heads] == 7.0)
    o_ref, lse_ref = R.mla_decode(case.q, case.kv_pool, case.page_table, case.lens)
    torch.testing.assert_close(wide[:, :heads].float().cpu(), o_ref, **O_TOL)
    torch.testing.assert_close(wide_lse[:, :heads].cpu(), lse_ref, **LSE_TOL)


@pytest.mark.parametrize("heads,ps,num_ctas", [(128, 32, 64), (192, 64, 7), (256, 128, 256)])
def test_decode_whole_head_groups(heads, ps, num_ctas):
    """Multiples of 64 heads on pages of >= 32 tokens: every 64-head group runs the warp-specialized
    kernel with its partials in its own workspace block; checked against the oracle, and the split
    step + merge entry points against the one-call entry point bit for bit."""
    print(f"[decode groups] heads={heads} ps={ps} ctas={num_ctas}", flush=True)
    case = make_decode_case(5, heads, ps, lens=[1, 700, 2049, 64, 4000], seed=heads + ps)
    check_case(case, num_ctas)
    B = len(case.lens)
    plan_np, slots = lib.decode_plan(case.lens, ps, num_ctas)
    plan = torch.from_numpy(plan_np).to(DEV)
    q, kv, pt, sl = case.q.to(DEV), case.kv_pool.to(DEV), case.page_table.to(DEV), case.seq_lens.to(DEV)
    outs = []
    for two_step in (False, True):
        ws_o, ws_lse = lib.decode_workspace(slots, heads, DEV)
        out = torch.empty((B, heads, 512), dtype=torch.bfloat16, device=DEV)
        lse = torch.empty((B, heads), dtype=torch.float32, device=DEV)
        lib.mla_decode(q, kv, pt, sl, plan, num_ctas, ws_o, ws_lse, R.DEFAULT_SCALE, out, lse, split_only=two_step)
        if two_step:
            lib.mla_decode_merge(ws_o, ws_lse, plan[num_ctas * 4 :], out, lse, single_piece_final=True)
        torch.cuda.synchronize()
        outs.append((out.cpu(), lse.cpu()))
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))
    assert torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("num_ctas", [256, 8])
def test_decode_many_short_requests(num_ctas):
    """1024 requests of 0..200 tokens: at 8 CTAs each CTA's range holds the plan's maximum of 128
    requests (the streaming kernel stages per-request bounds in LDS)."""
    print(f"[decode many] num_ctas={num_ctas}", flush=True)
    g = torch.Generator().manual_seed(21)
    lens = torch.randint(0, 201, (1024,), generator=g).tolist()
    case = make_decode_case(1024, 64, 64, lens=lens, seed=21)
    plan_np, _ = lib.decode_plan(lens, 64, num_ctas)
    cta = plan_np[: num_ctas * lib.PLAN_CTA_INTS].reshape(num_ctas, 4)
    per_cta = [min(int(re_) if ke == 0 else int(re_) + 1, 1024) - int(rb) for rb, _, re_, ke in cta]
    assert max(per_cta) <= lib.MAX_CTA_REQUESTS
    check_case(case, num_ctas)


def test_decode_kimi_k2_full_batch():
    """The benchmark's batch at full size: B=64, H=64, lengths U[1024, 8192], page 64, random pages."""
    case = make_decode_case(64, 64, 64, len_range=(1024, 8192), device=DEV, seed=0)
    out, lse, slots = run_decode(case.q, case.kv_pool, case.page_table, case.seq_lens, case.lens, 64, 256)
    assert slots > 0
    o_ref, lse_ref = R.mla_decode(case.q.cpu(), case.kv_pool.cpu(), case.page_table.cpu(), case.lens)
    torch.testing.assert_close(out, o_ref, **O_TOL)
    torch.testing.assert_close(lse, lse_ref, **LSE_TOL)


@pytest.mark.parametrize("num_ctas", [512, 1024])
def test_decode_kimi_k2_more_ranges_than_compute_units(num_ctas):
    """The benchmark's batch planned over 512 / 1024 CTA ranges (the warp-specialized kernel): the
    launch keeps one CTA per compute unit and each CTA runs its ranges w, w + 256, ... in turn."""
    case = make_decode_case(64, 64, 64, len_range=(1024, 8192), device=DEV, seed=4)
    out, lse, slots = run_decode(case.q, case.kv_pool, case.page_table, case.seq_lens, case.lens, 64, num_ctas)
    assert slots > 2 * 256
    o_ref, lse_ref = R.mla_decode(case.q.cpu(), case.kv_pool.cpu(), case.page_table.cpu(), case.lens)
    torch.testing.assert_close(out, o_ref, **O_TOL)
    torch.testing.assert_close(lse, lse_ref, **LSE_TOL)


@pytest.mark.parametrize("heads,ps", [(64, 64), (16, 1)])
def test_decode_padded_plan(heads, ps):
    """A plan made for 256 ranges laid out for 2048 (as for a captured graph): the kernels stop each
    CTA's loop at the first padding range; same bits as the unpadded plan."""
    from minisgl_amd.attention.mla import pad_plan

    case = make_decode_case(12, heads, ps, len_range=(1, 9000), device=DEV, seed=6)
    B = len(case.lens)
    plan_np, slots = lib.decode_plan(case.lens, ps, 256)
    outs = []
    for grid, pl in ((256, plan_np), (2048, pad_plan(plan_np, 256, 2048, B))):
        ws_o, ws_lse = lib.decode_workspace(slots, heads, DEV)
        out = torch.full((B, heads, 512), float("nan"), dtype=torch.bfloat16, device=DEV)
        lse = torch.full((B, heads), float("nan"), dtype=torch.float32, device=DEV)
        lib.mla_decode(case.q, case.kv_pool, case.page_table, case.seq_lens, torch.from_numpy(pl).to(DEV), grid,
                       ws_o, ws_lse, R.DEFAULT_SCALE, out, lse)
        torch.cuda.synchronize()
        outs.append((out.cpu(), lse.cpu()))
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))
    assert torch.equal(outs[0][1], outs[1][1])
    o_ref, lse_ref = R.mla_decode(case.q.cpu(), case.kv_pool.cpu(), case.page_table.cpu(), case.lens)
    torch.testing.assert_close(outs[0][0].float(), o_ref, **O_TOL)
    torch.testing.assert_close(outs[0][1], lse_ref, **LSE_TOL)


def test_decode_one_long_request_over_every_cta():
    """One 131072-token request split over all 256 CTAs: the merge reads 256 pieces per head."""
    case = make_decode_case(1, 64, 64, lens=[131072], seed=22)
    check_case(case, 256)


def test_decode_long_split_merge():
    """Long requests split over many CTAs exercise the LSE merge kernel."""
    case = make_decode_case(3, 64, 64, lens=[20000, 4097, 130], seed=3)
    check_case(case, 96)


def test_decode_empty_request():
    case = make_decode_case(3, 16, 16, lens=[5, 0, 100], seed=4)
    check_case(case, 16)


def test_decode_golden_fixture():
    f = np.load(os.path.join(HERE, "golden", "decode_small.npz"))
    bf = lambda a: torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)  # noqa: E731
    q, kv = bf(f["q_bits"]).to(DEV), bf(f["kv_bits"]).to(DEV)
    lens = f["seq_lens"].tolist()
    for ctas in (1, 3, 256):
        out, lse, _ = run_decode(q, kv, torch.from_numpy(f["page_table"]).to(DEV),
                                 torch.from_numpy(f["seq_lens"]).to(DEV), lens, int(f["page_size"]), ctas,
                                 float(f["scale"]))
        torch.testing.assert_close(out, torch.from_numpy(f["o"]), **O_TOL)
        torch.testing.assert_close(lse.double(), torch.from_numpy(f["lse"]), **LSE_TOL)


@pytest.mark.parametrize("heads,top", [(16, 30.0), (16, 90.0), (64, 90.0)])
def test_decode_large_logits(heads, top):
    """Scores that grow along the sequence by more than 2^64 force the exact-max rerun of a piece."""
    case = make_decode_case(2, heads, 64, lens=[900, 2000], seed=9)
    ramp = torch.linspace(0, top, case.kv_pool.shape[0] * 64).view(-1, 64, 1)
    kv = case.kv_pool.float()
    kv[..., 512:513] = ramp  # rope column grows with the flat row index
    case.kv_pool = kv.to(torch.bfloat16)
    case.q[..., 512] = 20.0
    check_case(case, 8)


@pytest.mark.parametrize("ps,num_ctas", [(32, 256), (128, 256), (64, 3), (32, 40)])
def test_decode_64_heads_page_sizes(ps, num_ctas):
    """64 heads with pages of >= 32 tokens (the streaming kernel), ragged lengths, many pieces per CTA."""
    case = make_decode_case(9, 64, ps, lens=[1, 33, 64, 96, 130, 255, 1000, 2049, 31], seed=ps)
    check_case(case, num_ctas)


def test_merge_kernel_standalone():
    """bf16 partials (in the chunk order of mla_amd.h), fp32 merge, one rounding to bf16: every output
    element lies within half a bf16 ulp of the float64 merge of those partials (plus fp32
    accumulation slack), so the merge rounds once and reads every dim from its chunk position."""
    gen = torch.Generator().manual_seed(5)
    H, S = 16, 11
    o_parts = torch.randn((S, H, 512), generator=gen).to(torch.bfloat16).double()  # the bf16 partials
    lse_parts = torch.randn((S, H), generator=gen) * 3
    lse_parts[4] = float("-inf")  # an empty piece
    req_info = torch.tensor([[0, 3, 0], [0, 1, 3], [0, 0, 0], [0, 7, 4]], dtype=torch.int32)
    out = torch.empty((4, H, 512), dtype=torch.bfloat16, device=DEV)
    lse = torch.empty((4, H), dtype=torch.float32, device=DEV)
    ws_o = o_parts[..., torch.from_numpy(lib.partial_chunk_dims())].to(torch.bfloat16)  # chunk order
    lib.mla_decode_merge(ws_o.to(DEV), lse_parts.to(DEV), req_info.flatten().to(DEV), out, lse)
    torch.cuda.synchronize()
    for b, (_, n, base) in enumerate(req_info.tolist()):
        o_ref, l_ref = R.mla_merge(o_parts[base : base + n].double(), lse_parts[base : base + n].double())
        # fp32 rounding in the weighted sum scales with sum_i w_i |o_i| (terms of either sign cancel)
        mag, _ = R.mla_merge(o_parts[base : base + n].double().abs(), lse_parts[base : base + n].double())
        got = out[b].double().cpu()
        exp = torch.floor(torch.log2(o_ref.abs().clamp_min(1e-30)))
        half_ulp = 2.0 ** (exp - 8)  # bf16 keeps 7 fraction bits
        err = (got - o_ref).abs()
        assert (err <= half_ulp + 2e-6 * mag + 1e-30).all(), f"request {b}: max err/half-ulp {(err / half_ulp).max():.3f}"
        torch.testing.assert_close(lse[b].double().cpu(), l_ref, atol=1e-5, rtol=1e-6)


@pytest.mark.parametrize("row_elems,index_dtype", [(576, torch.int32), (576, torch.int64), (64 * 192, torch.int32)])
def test_store_rows_bit_exact(row_elems, index_dtype):
    gen = torch.Generator().manual_seed(row_elems)
    rows = 4096
    cache = torch.randn((rows, row_elems), generator=gen).to(torch.bfloat16).to(DEV)
    before = cache.clone()
    for n in (1, 7, 64, 1000):
        idx = torch.randperm(rows, generator=gen)[:n].to(index_dtype)
        x = torch.randn((n, row_elems), generator=gen).to(torch.bfloat16).to(DEV)
        lib.store_rows(cache, idx.to(DEV), x)
        torch.cuda.synchronize()
        ref = before.cpu().clone()
        R.store_rows(ref, idx, x.cpu())
        assert torch.equal(cache.cpu().view(torch.int16), ref.view(torch.int16)), n
        before = cache.clone()


def test_page_table_kernel_bit_exact():
    f = np.load(os.path.join(HERE, "golden", "page_table_small.npz"))
    tt = torch.from_numpy(f["token_table"]).to(DEV)
    got = lib.page_table_from_tokens(tt, torch.from_numpy(f["table_idx"]).to(DEV), int(f["max_seqlen_k"]),
                                     int(f["page_size"]))
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), f["page_table"])
    # random tables at page sizes 1 and 64
    gen = torch.Generator().manual_seed(1)
    for ps in (1, 64):
        tt = torch.randint(0, 1 << 20, (9, 4096), generator=gen, dtype=torch.int32)
        idx = torch.randint(0, 9, (13,), generator=gen, dtype=torch.int32)
        ref = R.page_table_from_tokens(tt, idx, 4000, ps)
        got = lib.page_table_from_tokens(tt.to(DEV), idx.to(DEV), 4000, ps)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), ref)


@pytest.mark.parametrize("heads", [64, 128, 80])
def test_split_then_merge_equals_one_call(heads):
    """mla_decode_split_bf16 + mla_decode_merge_f32(single_piece_final) == mla_decode_bf16, bit for bit
    (more than 64 heads: groups of 64, each with its own block of the workspace)."""
    print(f"[split+merge] heads={heads}", flush=True)
    case = make_decode_case(6, heads, 64, lens=[5000, 70, 1, 3000, 129, 640], seed=11)
    q, kv, pt, sl = (t.to(DEV) for t in (case.q, case.kv_pool, case.page_table, case.seq_lens))
    plan_np, slots = lib.decode_plan(case.lens, 64, 32)
    plan = torch.from_numpy(plan_np).to(DEV)
    ws_o, ws_lse = lib.decode_workspace(slots, heads, DEV)
    outs = []
    for two_step in (False, True):
        out = torch.empty((6, heads, 512), dtype=torch.bfloat16, device=DEV)
        lse = torch.empty((6, heads), dtype=torch.float32, device=DEV)
        lib.mla_decode(q, kv, pt, sl, plan, 32, ws_o, ws_lse, R.DEFAULT_SCALE, out, lse, split_only=two_step)
        if two_step:
            lib.mla_decode_merge(ws_o, ws_lse, plan[32 * 4 :], out, lse, single_piece_final=True)
        torch.cuda.synchronize()
        outs.append((out.cpu(), lse.cpu()))
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))
    assert torch.equal(outs[0][1], outs[1][1])
    o_ref, lse_ref = R.mla_decode(case.q, case.kv_pool, case.page_table, case.lens)
    torch.testing.assert_close(outs[0][0].float(), o_ref, **O_TOL)
    torch.testing.assert_close(outs[0][1], lse_ref, **LSE_TOL)


def test_decode_long_context_split_kv():
    """Batch 8, 64 heads, lengths U[32768, 131072] (page_size 64): every request
    is split over many CTAs and merged through the fp32 LSE."""
    case = make_decode_case(8, 64, 64, len_range=(32768, 131072), device=DEV, seed=0)
    out, lse, slots = run_decode(case.q, case.kv_pool, case.page_table, case.seq_lens, case.lens, 64, 256)
    assert slots > 8  # split-KV really happened
    o_ref, lse_ref = R.mla_decode(case.q.cpu(), case.kv_pool.cpu(), case.page_table.cpu(), case.lens)
    torch.testing.assert_close(out, o_ref, **O_TOL)
    torch.testing.assert_close(lse, lse_ref, **LSE_TOL)


@pytest.mark.parametrize("ps", [1, 16, 64, 128])
def test_prefill_gather_bit_exact(ps):
    """mla_prefill_gather_bf16: every key's latent row (through the page table, any page size) lands
    bit for bit in its 64-row scratch page (latent dims and rope dims in their own row-strided
    buffers), rows past a request's keys stay untouched, and the scratch page table is
    seg_first[b] + i. Includes an empty request and page ids outside the pool (clamped)."""
    g = torch.Generator().manual_seed(ps)
    lens = [1, 64, 65, 0, 300, 129]
    pages = [-(-L // ps) for L in lens]
    num_pages = sum(pages) + 2
    pool = torch.randn((num_pages, ps, 576), generator=g).to(torch.bfloat16)
    width = max(max(pages), 1) + 1
    pt = torch.randint(0, num_pages, (len(lens), width), generator=g).to(torch.int32)
    pt[4, 0] = num_pages + 5  # out of range: clamped to the last page
    seg_pages = [-(-L // 64) for L in lens]
    seg_first = [0]
    for n in seg_pages[:-1]:
        seg_first.append(seg_first[-1] + n + 1)  # a gap page between requests
    rows = (seg_first[-1] + seg_pages[-1] + 1) * 64
    c = torch.full((rows, 520), 7.0, dtype=torch.bfloat16, device=DEV)  # row stride 520 > 512
    tail = torch.full((rows, 80), 7.0, dtype=torch.bfloat16, device=DEV)
    seg_pt = torch.full((len(lens), max(seg_pages) + 1), -1, dtype=torch.int32, device=DEV)
    lib.prefill_gather(pool.to(DEV), pt.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV),
                       torch.tensor(seg_first, dtype=torch.int32, device=DEV), max(seg_pages), c[:, :512],
                       tail[:, 8:72], seg_pt)
    torch.cuda.synchronize()
    c, tail, seg_pt = c.cpu(), tail.cpu(), seg_pt.cpu()
    flat = pool.reshape(-1, 576)
    written = torch.zeros(rows, dtype=torch.bool)
    for b, L in enumerate(lens):
        if L == 0:
            continue
        ptb = pt[b].clamp(0, num_pages - 1)
        src = flat[R.token_rows(ptb, L, ps)]
        dst = seg_first[b] * 64 + torch.arange(L)
        assert torch.equal(c[dst, :512].view(torch.int16), src[:, :512].view(torch.int16))
        assert torch.equal(tail[dst, 8:72].view(torch.int16), src[:, 512:].view(torch.int16))
        written[dst] = True
        assert seg_pt[b, : seg_pages[b]].tolist() == [seg_first[b] + i for i in range(seg_pages[b])]
    assert torch.all(c[~written] == 7.0) and torch.all(c[:, 512:] == 7.0)
    assert torch.all(tail[~written] == 7.0) and torch.all(tail[:, :8] == 7.0) and torch.all(tail[:, 72:] == 7.0)
    assert seg_pt[3].tolist() == [-1] * seg_pt.shape[1]  # the empty request writes no page


def _one_hot_targets(L, ps):
    """Token positions whose rows a one-hot query must gather: the first and last token, page
    edges, 32-token tile and 64-token plan-block edges, the 1024-page-id window edges, the last
    token of a partial tile, and a few inside (at most 64, one rope dim each)."""
    cand = [0, L - 1, ps - 1, ps, 2 * ps - 1, 31, 32, 63, 64, 65, 1023 * ps, 1024 * ps - 1, 1024 * ps,
            (L - 1) // 32 * 32 - 1, L // 2, L // 3, 5 * L // 7]
    out = []
    for t in cand:
        if 0 <= t < L and t not in out:
            out.append(t)
    return out[:64]


@pytest.mark.parametrize("ps", [1, 16, 64])
@pytest.mark.parametrize("num_ctas", [1, 7, 256])
def test_decode_one_hot_gather_bit_exact(ps, num_ctas):
    """A one-hot score makes every head's output the row it picks, bit for bit: target token k of
    request b carries rope dim 512 + k = 64 (all other rope dims 0), head h's query is 64 in rope dim
    h % n_b and 0 elsewhere, so its score is 64 * 64 / sqrt(192) = 295.6 for its target and 0 for
    every other token (e^-295 vanishes in fp32). A wrong page, row, tile or window in the kernel's
    gather shows up as a wrong row (the pattern of tests/kernel/test_index.py:52,91 in the
    reference: bit-exact gathers). Splits across CTAs are merged with the same weights 1 and 0."""
    H = 64
    lens = [1, 31, 33, 64, 65, 1000, 2500, 5000] if ps == 1 else [1, 33, 64, 65, 1000, 2500, 5000, 20000]
    print(f"[one-hot gather] ps={ps} ctas={num_ctas}", flush=True)
    case = make_decode_case(len(lens), H, ps, lens=lens, seed=ps + num_ctas)
    kv = case.kv_pool.clone()
    kv[..., 512:] = 0
    q = torch.zeros((len(lens), H, 576), dtype=torch.bfloat16)
    flat = kv.view(-1, 576)
    want = torch.empty((len(lens), H, 512), dtype=torch.bfloat16)
    for b, L in enumerate(lens):
        tg = _one_hot_targets(L, ps)
        rows = [int(case.page_table[b, t // ps]) * ps + t % ps for t in tg]
        for k, r in enumerate(rows):
            flat[r, 512 + k] = 64.0
        for h in range(H):
            k = h % len(tg)
            q[b, h, 512 + k] = 64.0
            want[b, h] = flat[rows[k], :512]
    out, lse, _ = run_decode(q.to(DEV), kv.to(DEV), case.page_table.to(DEV), case.seq_lens.to(DEV), lens, ps,
                             num_ctas)
    got = out.to(torch.bfloat16)
    bad = (got.view(torch.int16) != want.view(torch.int16)).any(-1)
    assert not bad.any(), f"rows gathered wrongly at (request, head) {bad.nonzero()[:8].tolist()}"
    s = 64.0 * 64.0 * R.DEFAULT_SCALE
    torch.testing.assert_close(lse, torch.full_like(lse, s), atol=1e-3, rtol=0.0)


@pytest.mark.parametrize("heads,ps", [(64, 1), (16, 1), (64, 2), (64, 16)])
@pytest.mark.parametrize("num_ctas", [1, 3])
def test_decode_long_pieces_small_pages(heads, ps, num_ctas):
    """Pieces longer than the general kernel's LDS window of 1024 page ids (page sizes under 32):
    the kernel restages the ids mid-piece; against the oracle."""
    print(f"[long pieces] heads={heads} ps={ps} ctas={num_ctas}", flush=True)
    lens = [5000, 1024 * ps + 17, 100, 2049]  # one CTA holds them all (at most 512 plan blocks)
    case = make_decode_case(len(lens), heads, ps, lens=lens, seed=heads + ps)
    plan_np, _ = lib.decode_plan(lens, ps, num_ctas)
    from minisgl_amd.attention.mla import plan_pieces

    longest = max(t1 - t0 for *_, t0, t1 in plan_pieces(plan_np, num_ctas, lens))
    assert num_ctas > 1 or longest > 1024 * ps, "one CTA takes the long request whole"
    check_case(case, num_ctas)


@pytest.mark.parametrize("ps,num_ctas", [(4, 256), (8, 5), (1, 9)])
def test_decode_64_heads_small_pages(ps, num_ctas):
    """64 heads with pages under 32 tokens (the streaming kernel with per-token row offsets): tiles
    that straddle pages, pieces shorter than a tile, lengths that are not multiples of 32."""
    case = make_decode_case(9, 64, ps, lens=[1, 33, 64, 96, 130, 255, 1000, 2049, 31], seed=100 + ps)
    check_case(case, num_ctas)


@pytest.mark.parametrize("ps", [1, 8])
def test_decode_large_logits_small_pages(ps):
    """The exact-max rerun of a piece with pages under 32 tokens: the rerun rewinds the stream, so
    the rewound tiles' row offsets are produced again."""
    case = make_decode_case(2, 64, ps, lens=[900, 2000], seed=19)
    ramp = torch.linspace(0, 90.0, case.kv_pool.shape[0] * ps).view(-1, ps, 1)
    kv = case.kv_pool.float()
    kv[..., 512:513] = ramp
    case.kv_pool = kv.to(torch.bfloat16)
    case.q[..., 512] = 20.0
    check_case(case, 8)


def test_decode_kimi_k2_page_size_one_more_ranges_than_compute_units():
    """The benchmark's batch at page size 1 (the reference's default), planned over 512 ranges: the
    streaming kernel with per-token row offsets, each CTA running two ranges in turn."""
    case = make_decode_case(64, 64, 1, len_range=(1024, 8192), device=DEV, seed=6)
    out, lse, slots = run_decode(case.q, case.kv_pool, case.page_table, case.seq_lens, case.lens, 1, 512)
    assert slots > 2 * 256
    o_ref, lse_ref = R.mla_decode(case.q.cpu(), case.kv_pool.cpu(), case.page_table.cpu(), case.lens)
    torch.testing.assert_close(out, o_ref, **O_TOL)
    torch.testing.assert_close(lse, lse_ref, **LSE_TOL)


def test_decode_small_pages_pool_beyond_32_bit_offsets():
    """A page-size-1 pool of more than 4 GiB: row offsets from the pool base no longer fit in 32
    bits, so 64 heads take the general kernel (64-bit row addresses); rows at the far end of the pool
    are read correctly."""
    pages = (1 << 32) // 1152 + 4096  # 4.0 GiB + 4.5 MiB of rows
    lens = [300, 77, 1500]
    g = torch.Generator().manual_seed(31)
    pool = torch.empty((pages, 1, 576), dtype=torch.bfloat16, device=DEV)
    pt = torch.zeros((3, 1500), dtype=torch.int32)
    used = torch.cat([torch.arange(pages - 2000, pages), torch.arange(0, 2000)])[torch.randperm(4000, generator=g)]
    off = 0
    for b, L in enumerate(lens):
        pt[b, :L] = used[off : off + L].to(torch.int32)
        off += L
    rows = torch.randn((4000, 1, 576), generator=g).to(torch.bfloat16)
    pool[pages - 2000 :] = rows[:2000].to(DEV)
    pool[:2000] = rows[2000:].to(DEV)
    q = torch.randn((3, 64, 576), generator=g).to(torch.bfloat16)
    small = torch.cat([rows[2000:], rows[:2000]])  # pool pages [0, 2000) then [pages - 2000, pages)
    # the oracle over the same rows, renumbered into a 4000-page pool
    remap = torch.full((pages,), -1, dtype=torch.int64)
    remap[:2000] = torch.arange(2000)
    remap[pages - 2000 :] = torch.arange(2000, 4000)
    pt_small = remap[pt.long()].to(torch.int32)
    pt_small[pt_small < 0] = 0
    o_ref, lse_ref = R.mla_decode(q, small, pt_small, lens)
    out, lse, _ = run_decode(q.to(DEV), pool, pt.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV), lens,
                             1, 256)
    del pool
    torch.testing.assert_close(out, o_ref, **O_TOL)
    torch.testing.assert_close(lse, lse_ref, **LSE_TOL)
