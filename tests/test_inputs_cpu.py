"""Structure of the seeded benchmark inputs (CPU only): shared-prefix page
tables of the mixed ragged batch."""

from __future__ import annotations

import torch

from minisgl_amd.benchmark.inputs import make_mixed_case


def test_mixed_case_page_sharing():
    ps, groups, prefix = 64, 3, 256
    m = make_mixed_case(8, 4, 2, ps, (100, 1000), 150, prefix, groups, seed=4)
    pp = prefix // ps
    d, p = m.decode, m.prefill
    rows = {}
    for b, L in enumerate(d.lens):
        n = -(-L // ps)
        rows[("d", b)] = (m.group_of_decode[b], d.page_table[b, :n].tolist())
    for i, E in enumerate(p.extends):
        n = -(-(prefix + E) // ps)
        rows[("p", i)] = (m.group_of_prefill[i], p.page_table[i, :n].tolist())
    prefixes = {}
    owned = []
    for key, (g, ids) in rows.items():
        k = min(pp, len(ids))
        ref = prefixes.setdefault(g, None)
        if ref is None or len(ref) < k:
            prefixes[g] = ids[:k] if ref is None or ids[: len(ref)] == ref else None
        assert prefixes[g] is not None and ids[:k] == prefixes[g][:k], f"{key} does not share its group prefix"
        owned += ids[k:]
    # private pages are unique, disjoint from every shared prefix
    shared = {i for ids in prefixes.values() for i in ids}
    assert len(owned) == len(set(owned)) and not (set(owned) & shared)
    # a prefill chunk's pages are all inside the per-head pools, every page inside the latent pool
    assert int(p.page_table.max()) < p.k_pool.shape[0] == p.v_pool.shape[0]
    assert int(d.page_table.max()) < d.kv_pool.shape[0]
    assert p.seq_lens_k.tolist() == [prefix + E for E in p.extends]
    assert torch.equal(p.cu_seqlens_q, torch.tensor([0, 150, 300, 450, 600], dtype=torch.int32))
