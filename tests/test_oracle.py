"""Pins for the CPU oracle (oracle/ref_mla.py), run on the CPU.

Each check is chosen so a plausible mistake fails it: float64 pure-Python
loops, closed forms, torch's own SDPA routine, split/merge equivalence and the
absorbed-vs-decompressed MLA identity. ``test_planted_mistakes_are_caught``
re-runs the pins against deliberately broken copies of the oracle and asserts
each copy is rejected.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import ref_mla as R

torch.set_num_threads(min(8, torch.get_num_threads()))


# ----------------------------------------------------------------------------- helpers
def _paged_pool(num_pages, ps, row_shape, gen, dtype=torch.bfloat16):
    return torch.randn((num_pages, ps) + tuple(row_shape), generator=gen).to(dtype)


def _random_page_table(lens, ps, num_pages, gen):
    need = [max(1, -(-L // ps)) for L in lens]
    perm = torch.randperm(num_pages, generator=gen)
    assert sum(need) <= num_pages
    width = max(need)
    pt = torch.zeros((len(lens), width), dtype=torch.int32)
    off = 0
    for b, n in enumerate(need):
        pt[b, :n] = perm[off : off + n].to(torch.int32)
        off += n
    return pt


def _decode_case(B=3, H=4, lens=(1, 5, 9), ps=4, seed=0):
    gen = torch.Generator().manual_seed(seed)
    num_pages = sum(-(-L // ps) for L in lens) + 3
    pool = _paged_pool(num_pages, ps, (R.KV_DIM,), gen)
    pt = _random_page_table(lens, ps, num_pages, gen)
    q = torch.randn((B, H, R.KV_DIM), generator=gen).to(torch.bfloat16)
    return q, pool, pt, list(lens)


def _loops_decode(q, pool, pt, lens, scale, dv=R.LATENT_DIM):
    """float64 pure-Python loops: no matmul, no logsumexp."""
    B, H, D = q.shape
    ps = pool.shape[1]
    o = [[[0.0] * dv for _ in range(H)] for _ in range(B)]
    lse = [[float("-inf")] * H for _ in range(B)]
    for b in range(B):
        rows = []
        for t in range(lens[b]):
            page = int(pt[b, t // ps])
            rows.append(pool[page, t % ps].double().tolist())
        for h in range(H):
            qv = q[b, h].double().tolist()
            s = [scale * sum(qv[d] * r[d] for d in range(D)) for r in rows]
            if not s:
                continue
            m = max(s)
            e = [math.exp(x - m) for x in s]
            z = sum(e)
            lse[b][h] = m + math.log(z)
            for d in range(dv):
                o[b][h][d] = sum(e[t] * rows[t][d] for t in range(len(rows))) / z
    return torch.tensor(o, dtype=torch.float64), torch.tensor(lse, dtype=torch.float64)


# ----------------------------------------------------------------------------- decode pins
def check_decode_pins(decode) -> bool:
    """True when ``decode`` (same signature as ``R.mla_decode``) passes every pin."""
    ok = True
    scale = R.DEFAULT_SCALE
    # 1. float64 brute force on a tiny ragged batch (includes L=1 and a partial page)
    q, pool, pt, lens = _decode_case()
    o, lse = decode(q, pool, pt, lens, scale, dtype=torch.float64)
    o_ref, lse_ref = _loops_decode(q, pool, pt, lens, scale)
    ok &= torch.allclose(o, o_ref, atol=1e-10, rtol=1e-10)
    ok &= torch.allclose(lse, lse_ref, atol=1e-10, rtol=1e-10)
    # 2. one key: o = kv[:512], lse = s
    q1, pool1, pt1, _ = _decode_case(B=1, H=2, lens=(1,), ps=1, seed=3)
    o, lse = decode(q1, pool1, pt1, [1], scale, dtype=torch.float64)
    kv = pool1[int(pt1[0, 0]), 0].double()
    ok &= torch.allclose(o[0], kv[: R.LATENT_DIM].expand(2, -1), atol=1e-12)
    ok &= torch.allclose(lse[0], scale * (q1[0].double() @ kv), atol=1e-10)
    # 3. equal scores (q = 0): o = mean of values, lse = ln L
    q0 = torch.zeros_like(q)
    o, lse = decode(q0, pool, pt, lens, scale, dtype=torch.float64)
    for b, L in enumerate(lens):
        rows = R.gather_rows(pool.reshape(-1, R.KV_DIM), pt[b], L, pool.shape[1]).double()
        ok &= torch.allclose(o[b], rows[:, : R.LATENT_DIM].mean(0).expand_as(o[b]), atol=1e-10)
        ok &= torch.allclose(lse[b], torch.full_like(lse[b], math.log(L)), atol=1e-12)
    # 4. dominant key: q aligned with one token's rope part, scaled up
    b, L = 2, lens[2]
    rows = R.gather_rows(pool.reshape(-1, R.KV_DIM), pt[b], L, pool.shape[1]).double()
    target = 6
    qd = torch.zeros_like(q)
    qd[b, :, R.LATENT_DIM:] = (rows[target, R.LATENT_DIM:] * 40.0).to(torch.bfloat16)
    o, _ = decode(qd, pool, pt, lens, scale, dtype=torch.float64)
    ok &= torch.allclose(o[b], rows[target, : R.LATENT_DIM].expand_as(o[b]), atol=1e-6)
    # 5. score shift: constant rope column c on every key, shift q's rope dim by delta
    pool_c = pool.clone()
    pool_c[..., R.LATENT_DIM] = 2.0
    delta = 3.0
    q_s = q.clone()
    q_s[..., R.LATENT_DIM] = (q_s[..., R.LATENT_DIM].float() + delta).to(torch.bfloat16)
    o_a, lse_a = decode(q, pool_c, pt, lens, scale, dtype=torch.float64)
    o_b, lse_b = decode(q_s, pool_c, pt, lens, scale, dtype=torch.float64)
    shift = scale * 2.0 * (q_s[..., R.LATENT_DIM].double() - q[..., R.LATENT_DIM].double())
    ok &= torch.allclose(o_a, o_b, atol=1e-10)
    ok &= torch.allclose(lse_b - lse_a, shift, atol=1e-10)
    # 6. torch SDPA (library routine) on the gathered keys
    for b, L in enumerate(lens):
        rows = R.gather_rows(pool.reshape(-1, R.KV_DIM), pt[b], L, pool.shape[1]).double()
        ref = torch.nn.functional.scaled_dot_product_attention(
            q[b].double().unsqueeze(1), rows.unsqueeze(0), rows[:, : R.LATENT_DIM].unsqueeze(0), scale=scale
        )[:, 0]
        o, _ = decode(q, pool, pt, lens, scale, dtype=torch.float64)
        ok &= torch.allclose(o[b], ref, atol=1e-10)
    return bool(ok)


def test_decode_pins():
    assert check_decode_pins(R.mla_decode)


def test_decode_fp32_close_to_fp64():
    q, pool, pt, lens = _decode_case(B=4, H=8, lens=(1, 63, 64, 200), ps=16, seed=5)
    o32, l32 = R.mla_decode(q, pool, pt, lens)
    o64, l64 = R.mla_decode(q, pool, pt, lens, dtype=torch.float64)
    assert torch.allclose(o32.double(), o64, atol=1e-5, rtol=1e-5)
    assert torch.allclose(l32.double(), l64, atol=1e-5)


def test_decode_empty_request():
    q, pool, pt, _ = _decode_case(B=2, H=2, lens=(3, 4), ps=4)
    o, lse = R.mla_decode(q, pool, pt, [0, 4])
    assert torch.all(o[0] == 0) and torch.all(torch.isneginf(lse[0]))
    assert torch.all(torch.isfinite(lse[1]))


# ----------------------------------------------------------------------------- merge pins
def _split_points(L, n, gen):
    if n <= 1 or L <= 1:
        return [0, L]
    cuts = sorted(torch.randperm(L - 1, generator=gen)[: n - 1].add(1).tolist())
    return [0] + cuts + [L]


def check_merge_pins(merge) -> bool:
    ok = True
    gen = torch.Generator().manual_seed(11)
    q, pool, pt, lens = _decode_case(B=3, H=4, lens=(7, 33, 90), ps=8, seed=2)
    o_full, lse_full = R.mla_decode(q, pool, pt, lens, dtype=torch.float64)
    for b, L in enumerate(lens):
        for nsplit in (1, 2, 5):
            pts = _split_points(L, nsplit, gen)
            pieces = [(b, pts[i], pts[i + 1]) for i in range(len(pts) - 1)]
            o_p, l_p = R.mla_decode_pieces(q, pool, pt, pieces, dtype=torch.float64)
            o_m, l_m = merge(o_p, l_p)
            ok &= torch.allclose(o_m, o_full[b], atol=1e-10)
            ok &= torch.allclose(l_m, lse_full[b], atol=1e-10)
            perm = torch.randperm(len(pieces), generator=gen)
            o_m2, l_m2 = merge(o_p[perm], l_p[perm])
            ok &= torch.allclose(o_m2, o_m, atol=1e-12) and torch.allclose(l_m2, l_m, atol=1e-12)
        # an empty piece contributes nothing
        pieces = [(b, 0, L), (b, L, L)]
        o_p, l_p = R.mla_decode_pieces(q, pool, pt, pieces, dtype=torch.float64)
        o_m, l_m = merge(o_p, l_p)
        ok &= torch.allclose(o_m, o_full[b], atol=1e-12) and torch.allclose(l_m, lse_full[b], atol=1e-12)
    return bool(ok)


def test_merge_pins():
    assert check_merge_pins(R.mla_merge)


def test_merge_all_empty():
    o, lse = R.mla_merge(torch.zeros(3, 2, 8), torch.full((3, 2), float("-inf")))
    assert torch.all(o == 0) and torch.all(torch.isneginf(lse))


# ----------------------------------------------------------------------------- prefill pins
def _prefill_case(H=3, extends=(5, 4), prefixes=(0, 6), ps=4, dqk=R.PREFILL_QK_DIM, dv=R.PREFILL_V_DIM, seed=0):
    gen = torch.Generator().manual_seed(seed)
    lens = [p + e for p, e in zip(prefixes, extends)]
    num_pages = sum(-(-L // ps) for L in lens) + 2
    kp = _paged_pool(num_pages, ps, (H, dqk), gen)
    vp = _paged_pool(num_pages, ps, (H, dv), gen)
    pt = _random_page_table(lens, ps, num_pages, gen)
    cu = [0]
    for e in extends:
        cu.append(cu[-1] + e)
    q = torch.randn((cu[-1], H, dqk), generator=gen).to(torch.bfloat16)
    return q, kp, vp, pt, cu, lens


def _loops_prefill(q, kp, vp, pt, cu, lens, scale):
    T, H, D = q.shape
    ps = kp.shape[1]
    dv = vp.shape[-1]
    o = torch.zeros((T, H, dv), dtype=torch.float64)
    lse = torch.full((T, H), float("-inf"), dtype=torch.float64)
    for b in range(len(lens)):
        E = cu[b + 1] - cu[b]
        L = lens[b]
        for i in range(E):
            pos = L - E + i
            for h in range(H):
                qv = q[cu[b] + i, h].double()
                s, vs = [], []
                for j in range(pos + 1):
                    page = int(pt[b, j // ps])
                    s.append(scale * float(qv @ kp[page, j % ps, h].double()))
                    vs.append(vp[page, j % ps, h].double())
                m = max(s)
                e = [math.exp(x - m) for x in s]
                z = sum(e)
                lse[cu[b] + i, h] = m + math.log(z)
                o[cu[b] + i, h] = sum(w * v for w, v in zip(e, vs)) / z
    return o, lse


def check_prefill_pins(prefill) -> bool:
    ok = True
    scale = R.DEFAULT_SCALE
    # 1. brute force, with and without a prefix, partial pages
    q, kp, vp, pt, cu, lens = _prefill_case()
    o, lse = prefill(q, kp, vp, pt, cu, lens, scale, dtype=torch.float64)
    o_ref, lse_ref = _loops_prefill(q, kp, vp, pt, cu, lens, scale)
    ok &= torch.allclose(o, o_ref, atol=1e-10) and torch.allclose(lse, lse_ref, atol=1e-10)
    # 2. no prefix: torch SDPA with is_causal=True
    q, kp, vp, pt, cu, lens = _prefill_case(H=2, extends=(9,), prefixes=(0,), seed=4)
    o, _ = prefill(q, kp, vp, pt, cu, lens, scale, dtype=torch.float64)
    rows = R.token_rows(pt[0], lens[0], kp.shape[1])
    k = kp.reshape(-1, 2, R.PREFILL_QK_DIM)[rows].double().transpose(0, 1)
    v = vp.reshape(-1, 2, R.PREFILL_V_DIM)[rows].double().transpose(0, 1)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.double().transpose(0, 1), k, v, is_causal=True, scale=scale
    ).transpose(0, 1)
    ok &= torch.allclose(o, ref, atol=1e-10)
    # 3. extend of one token over a prefix sees every key (decode in decompressed form)
    q, kp, vp, pt, cu, lens = _prefill_case(H=2, extends=(1,), prefixes=(10,), seed=6)
    o, _ = prefill(q, kp, vp, pt, cu, lens, scale, dtype=torch.float64)
    rows = R.token_rows(pt[0], lens[0], kp.shape[1])
    k = kp.reshape(-1, 2, R.PREFILL_QK_DIM)[rows].double().transpose(0, 1)
    v = vp.reshape(-1, 2, R.PREFILL_V_DIM)[rows].double().transpose(0, 1)
    ref = torch.nn.functional.scaled_dot_product_attention(q.double().transpose(0, 1), k, v, scale=scale)
    ok &= torch.allclose(o, ref.transpose(0, 1), atol=1e-10)
    return bool(ok)


def test_prefill_pins():
    assert check_prefill_pins(R.mla_prefill)


def test_absorbed_equals_decompressed():
    """q_nope.(W_UK c) == (W_UK^T q_nope).c and (sum p c) W_UV == sum p (c W_UV): ties decode to prefill."""
    gen = torch.Generator().manual_seed(21)
    H, L, ps = 3, 11, 4
    c = torch.randn((L, R.LATENT_DIM), generator=gen, dtype=torch.float64)
    k_pe = torch.randn((L, R.ROPE_DIM), generator=gen, dtype=torch.float64)
    w_uk = torch.randn((H, 128, R.LATENT_DIM), generator=gen, dtype=torch.float64) / 16
    w_uv = torch.randn((H, R.LATENT_DIM, 128), generator=gen, dtype=torch.float64) / 16
    q_nope = torch.randn((H, 128), generator=gen, dtype=torch.float64)
    q_pe = torch.randn((H, R.ROPE_DIM), generator=gen, dtype=torch.float64)
    pages = -(-L // ps)
    pt = torch.arange(pages, dtype=torch.int32).flip(0).unsqueeze(0)
    # absorbed: latent pool + 576-wide q
    latent = torch.zeros((pages * ps, R.KV_DIM), dtype=torch.float64)
    rows = R.token_rows(pt[0], L, ps)
    latent[rows] = torch.cat([c, k_pe], dim=1)
    q_abs = torch.cat([torch.einsum("hk,hkd->hd", q_nope, w_uk), q_pe], dim=1).unsqueeze(0)
    o_lat, lse_a = R.mla_decode(q_abs, latent.view(pages, ps, -1), pt, [L], dtype=torch.float64)
    o_abs = torch.einsum("hd,hdv->hv", o_lat[0], w_uv)
    # decompressed: per-head K (128 nope + 64 rope) and V (128), one-token extend
    k_heads = torch.cat([torch.einsum("hkd,ld->lhk", w_uk, c), k_pe.unsqueeze(1).expand(L, H, -1)], dim=2)
    v_heads = torch.einsum("ld,hdv->lhv", c, w_uv)
    kp = torch.zeros((pages * ps, H, R.PREFILL_QK_DIM), dtype=torch.float64)
    vp = torch.zeros((pages * ps, H, R.PREFILL_V_DIM), dtype=torch.float64)
    kp[rows], vp[rows] = k_heads, v_heads
    q_dec = torch.cat([q_nope, q_pe], dim=1).unsqueeze(0)
    o_dec, lse_d = R.mla_prefill(
        q_dec, kp.view(pages, ps, H, -1), vp.view(pages, ps, H, -1), pt, [0, 1], [L], dtype=torch.float64
    )
    assert torch.allclose(o_abs, o_dec[0], atol=1e-9)
    assert torch.allclose(lse_a[0], lse_d[0], atol=1e-9)


def test_decompress_pool_scalar_loops():
    """decompress_pool against float64 loops: K[t, h, d] = sum_i kv_b[256h + d, i] c_t[i] (d < 128),
    K[t, h, 128 + r] = k_pe_t[r], V[t, h, d] = sum_i kv_b[256h + 128 + d, i] c_t[i]."""
    gen = torch.Generator().manual_seed(23)
    H, pages, ps = 2, 2, 2
    pool = torch.randn((pages, ps, R.KV_DIM), generator=gen, dtype=torch.float64)
    kv_b = torch.randn((H * 256, R.LATENT_DIM), generator=gen, dtype=torch.float64)
    K, V = R.decompress_pool(pool, kv_b, H)
    for p in range(pages):
        for t in range(ps):
            row = pool[p, t].tolist()
            for h in (0, H - 1):
                for d in (0, 77, 127):
                    kn = sum(float(kv_b[256 * h + d, i]) * row[i] for i in range(R.LATENT_DIM))
                    vv = sum(float(kv_b[256 * h + 128 + d, i]) * row[i] for i in range(R.LATENT_DIM))
                    assert abs(float(K[p, t, h, d]) - kn) < 1e-9 and abs(float(V[p, t, h, d]) - vv) < 1e-9
                for r in (0, 63):
                    assert float(K[p, t, h, 128 + r]) == row[R.LATENT_DIM + r]


def test_decompress_pool_prefill_equals_absorbed_decode():
    """A one-token extend over decompress_pool's pages equals absorbed decode over the latent pool
    with q_abs = [q_nope W_UK | q_pe] and o = o_lat W_UV^T: ties the decompression to decode."""
    gen = torch.Generator().manual_seed(29)
    H, L, ps = 3, 13, 4
    pages = -(-L // ps) + 1
    pool = torch.randn((pages, ps, R.KV_DIM), generator=gen, dtype=torch.float64)
    kv_b = torch.randn((H * 256, R.LATENT_DIM), generator=gen, dtype=torch.float64) / 16
    pt = torch.randperm(pages, generator=gen)[: -(-L // ps)].to(torch.int32).unsqueeze(0)
    q = torch.randn((1, H, R.PREFILL_QK_DIM), generator=gen, dtype=torch.float64)
    K, V = R.decompress_pool(pool, kv_b, H)
    o_dec, lse_d = R.mla_prefill(q, K, V, pt, [0, 1], [L], dtype=torch.float64)
    w = kv_b.view(H, 2, 128, R.LATENT_DIM)
    q_abs = torch.cat([torch.einsum("hk,hkl->hl", q[0, :, :128], w[:, 0]), q[0, :, 128:]], dim=1).unsqueeze(0)
    o_lat, lse_a = R.mla_decode(q_abs, pool, pt, [L], dtype=torch.float64)
    o_abs = torch.einsum("hl,hdl->hd", o_lat[0], w[:, 1])
    assert torch.allclose(o_abs, o_dec[0], atol=1e-9)
    assert torch.allclose(lse_a[0], lse_d[0], atol=1e-9)


# ----------------------------------------------------------------------------- page table / store pins
def _loops_page_table(token_table, table_idx, max_len, ps):
    out = []
    for r in table_idx.tolist():
        out.append([int(token_table[r, j]) // ps for j in range(0, max_len, ps)])
    return torch.tensor(out, dtype=torch.int32)


def _allocate_token_table(rows, width, ps, num_pages, lens, gen):
    """Token table as the reference's CacheManager writes it (scheduler/cache.py:119-146)."""
    tt = torch.zeros((rows, width), dtype=torch.int32)
    free = (torch.randperm(num_pages, generator=gen) * ps).to(torch.int32)
    off = 0
    for r, L in enumerate(lens):
        n = -(-L // ps)
        pages = free[off : off + n]
        off += n
        toks = (pages.unsqueeze(1) + torch.arange(ps, dtype=torch.int32)).flatten()
        tt[r, : n * ps] = toks
    return tt


@pytest.mark.parametrize("ps", [1, 16, 64])
def test_page_table_conversion(ps):
    gen = torch.Generator().manual_seed(ps)
    lens = [1, ps + 1, 3 * ps, 7 * ps - 1]
    width = 8 * ps
    tt = _allocate_token_table(6, width, ps, 64, lens, gen)
    idx = torch.tensor([3, 0, 2, 1], dtype=torch.int32)
    max_len = max(lens[i] for i in idx.tolist())
    got = R.page_table_from_tokens(tt, idx, max_len, ps)
    assert got.dtype == torch.int32 and got.shape == (4, -(-max_len // ps))
    assert torch.equal(got, _loops_page_table(tt, idx, max_len, ps))
    # invariants of the token table (tests/core/test_cache_allocate.py:147-169): page-aligned starts,
    # consecutive tokens inside a page, so gathering via the page table reproduces the token table
    for b, r in enumerate(idx.tolist()):
        L = lens[r]
        assert torch.all(tt[r, :L:ps] % ps == 0)
        rows = R.token_rows(got[b], L, ps)
        assert torch.equal(rows.to(torch.int32), tt[r, :L])


def test_store_rows_bit_exact():
    gen = torch.Generator().manual_seed(7)
    cache = torch.randn((256, R.KV_DIM), generator=gen).to(torch.bfloat16)
    before = cache.clone()
    idx = torch.randperm(256, generator=gen)[:40].to(torch.int32)
    x = torch.randn((40, R.KV_DIM), generator=gen).to(torch.bfloat16)
    R.store_rows(cache, idx, x)
    for i, r in enumerate(idx.tolist()):
        assert torch.equal(cache[r].view(torch.int16), x[i].view(torch.int16))
    untouched = torch.ones(256, dtype=torch.bool)
    untouched[idx.long()] = False
    assert torch.equal(cache[untouched].view(torch.int16), before[untouched].view(torch.int16))


# ----------------------------------------------------------------------------- planted mistakes
def _mutant_decode(kind):
    def decode(q, pool, pt, lens, scale=R.DEFAULT_SCALE, *, dv=R.LATENT_DIM, dtype=torch.float32):
        if kind == "scale":
            return R.mla_decode(q, pool, pt, lens, scale * 1.01, dv=dv, dtype=dtype)
        if kind == "drop_rope":
            q2 = q.clone()
            q2[..., R.LATENT_DIM :] = 0
            return R.mla_decode(q2, pool, pt, lens, scale, dv=dv, dtype=dtype)
        if kind == "log2":
            o, lse = R.mla_decode(q, pool, pt, lens, scale, dv=dv, dtype=dtype)
            return o, lse / math.log(2.0)
        if kind == "off_by_one":  # drops the newest token
            return R.mla_decode(q, pool, pt, [max(1, L - 1) for L in lens], scale, dv=dv, dtype=dtype)
        if kind == "page_order":  # reads pages in reverse order
            pt2 = pt.clone()
            for b, L in enumerate(lens):
                n = -(-L // pool.shape[1])
                pt2[b, :n] = pt[b, :n].flip(0)
            return R.mla_decode(q, pool, pt2, lens, scale, dv=dv, dtype=dtype)
        if kind == "value_offset":  # values taken from dims 64..575
            B, H, _ = q.shape
            o = torch.zeros((B, H, dv), dtype=dtype)
            lse = torch.zeros((B, H), dtype=dtype)
            flat = pool.reshape(-1, R.KV_DIM)
            for b, L in enumerate(lens):
                kv = R.gather_rows(flat, pt[b], L, pool.shape[1]).to(dtype)
                s = (q[b].to(dtype) @ kv.T) * scale
                lse[b] = torch.logsumexp(s, -1)
                o[b] = torch.softmax(s, -1) @ kv[:, 64 : 64 + dv]
            return o, lse
        raise ValueError(kind)

    return decode


def _mutant_merge(kind):
    def merge(o_parts, lse_parts):
        if kind == "no_weights":
            return o_parts.mean(0), torch.logsumexp(lse_parts, 0)
        if kind == "max_lse":
            o, _ = R.mla_merge(o_parts, lse_parts)
            return o, lse_parts.max(0).values
        raise ValueError(kind)

    return merge


def _mutant_prefill(kind):
    def prefill(q, kp, vp, pt, cu, lens, scale=R.DEFAULT_SCALE, *, dtype=torch.float32):
        if kind == "top_left_causal":  # query i sees keys j <= i (ignores the prefix)
            lens2 = [cu[b + 1] - cu[b] for b in range(len(lens))]
            return R.mla_prefill(q, kp, vp, pt, cu, lens2, scale, dtype=dtype)
        if kind == "no_mask":
            T, H, _ = q.shape
            o = torch.zeros((T, H, vp.shape[-1]), dtype=dtype)
            lse = torch.zeros((T, H), dtype=dtype)
            for b, L in enumerate(lens):
                rows = R.token_rows(pt[b], L, kp.shape[1])
                k = kp.reshape(-1, H, kp.shape[-1])[rows].to(dtype).transpose(0, 1)
                v = vp.reshape(-1, H, vp.shape[-1])[rows].to(dtype).transpose(0, 1)
                qb = q[cu[b] : cu[b + 1]].to(dtype).transpose(0, 1)
                s = qb @ k.transpose(1, 2) * scale
                o[cu[b] : cu[b + 1]] = (torch.softmax(s, -1) @ v).transpose(0, 1)
                lse[cu[b] : cu[b + 1]] = torch.logsumexp(s, -1).transpose(0, 1)
            return o, lse
        raise ValueError(kind)

    return prefill


@pytest.mark.parametrize("kind", ["scale", "drop_rope", "log2", "off_by_one", "page_order", "value_offset"])
def test_planted_decode_mistakes_are_caught(kind):
    assert not check_decode_pins(_mutant_decode(kind))


@pytest.mark.parametrize("kind", ["no_weights", "max_lse"])
def test_planted_merge_mistakes_are_caught(kind):
    assert not check_merge_pins(_mutant_merge(kind))


@pytest.mark.parametrize("kind", ["top_left_causal", "no_mask"])
def test_planted_prefill_mistakes_are_caught(kind):
    assert not check_prefill_pins(_mutant_prefill(kind))
