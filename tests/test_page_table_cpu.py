"""The token-table writer (page-granular allocation, python/minisgl/scheduler/cache.py) on the
CPU: its invariants are the reference's own (tests/core/test_cache_allocate.py: page-aligned
free slots, no overlapping pages, consecutive tokens inside a page) plus the page-table closed
form the backend relies on (oracle/ref_mla.py page_table_from_tokens)."""

from __future__ import annotations

import pytest
import torch

from minisgl_amd.core import Req
from minisgl_amd.kvcache import PagedTokenTable
from oracle import ref_mla as R


def _check_rows(pt: PagedTokenTable, lens):
    ps = pt.page_size
    seen = set()
    for r, L in lens.items():
        toks = pt.page_table[r, : -(-L // ps) * ps].tolist()
        for p in range(0, len(toks), ps):
            start = toks[p]
            assert start % ps == 0, "page starts are page-aligned"
            assert toks[p : p + ps] == list(range(start, start + ps)), "tokens inside a page are consecutive"
            assert start not in seen, "no page is given twice"
            seen.add(start)
        # the backend's page table: new_pt[b, j] = tok[b, j * ps] // ps
        pages = R.page_table_from_tokens(pt.page_table, torch.tensor([r], dtype=torch.int32), L, ps)[0]
        assert pages.tolist() == [toks[j * ps] // ps for j in range(-(-L // ps))]


@pytest.mark.parametrize("ps", [1, 4, 64])
def test_allocate_grow_free_reuse(ps):
    num_pages = 600 // ps + 20
    tt = torch.full((6, 512), -1, dtype=torch.int32)
    pt = PagedTokenTable(num_pages, ps, tt)
    reqs = [Req(table_idx=i, cached_len=0, device_len=L) for i, L in enumerate([70, 1, 129, 64])]
    pt.allocate_paged(reqs)
    lens = {r.table_idx: r.device_len for r in reqs}
    _check_rows(pt, lens)
    # out_loc = the new positions' token locations, in batch order
    assert torch.equal(pt.out_loc(reqs), torch.cat([tt[r.table_idx, : r.device_len] for r in reqs]))
    # decode growth: a new page only when a request crosses a page boundary
    before = pt.free_pages
    for r in reqs:
        r.complete_one()
    pt.allocate_paged(reqs)
    crossing = sum(1 for r in reqs if -(-r.device_len // ps) > -(-r.cached_len // ps))
    assert before - pt.free_pages == crossing
    lens = {r.table_idx: r.device_len for r in reqs}
    _check_rows(pt, lens)
    # a finished request frees its pages; a new request reuses them (non-contiguous rows)
    pt.free(2, lens.pop(2))
    new = Req(table_idx=4, cached_len=0, device_len=200)
    pt.allocate_paged([new])
    lens[4] = 200
    _check_rows(pt, lens)
    used = sum(-(-L // ps) for L in lens.values())
    assert pt.free_pages + used == num_pages


def test_out_of_pages_raises():
    pt = PagedTokenTable(2, 64, torch.zeros((2, 256), dtype=torch.int32))
    with pytest.raises(RuntimeError, match="out of KV pages"):
        pt.allocate_paged([Req(table_idx=0, cached_len=0, device_len=129)])
    assert pt.free_pages == 2
