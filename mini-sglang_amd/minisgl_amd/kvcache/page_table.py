"""Page-granular writer of the token table that the MLA backend reads.

Mirrors the page half of the reference's ``CacheManager`` (python/minisgl/scheduler/cache.py):
``allocate_paged`` (:42-53), ``_allocate`` / ``_free`` (:119-131), ``_page_to_token`` (:133-139)
and ``_write_page_table`` (:142-161). Free pages are kept as page-aligned token offsets; a
request growing from ``cached_len`` to ``device_len`` receives the pages
``ceil(cached_len / ps) .. ceil(device_len / ps) - 1`` of its row, and page ``p`` of the row
gets the tokens ``page_start + j`` (``j < ps``): tokens inside a page are consecutive, pages are
taken in free-list order, so after frees a row's pages are not contiguous. The backend turns
this token table into its page table (``mla_page_table_from_tokens``).

The radix prefix cache and its eviction are outside the attention path and not built: asking
for more pages than are free raises.
"""

from __future__ import annotations

from typing import Iterable, List, Tuple

import torch


class PagedTokenTable:
    def __init__(self, num_pages: int, page_size: int, page_table: torch.Tensor) -> None:
        assert page_table.dtype == torch.int32 and page_table.dim() == 2
        self.page_table = page_table  # [max_running_req + 1, max_seq_len] token locations
        self.page_size = page_size
        self.num_pages = num_pages
        self.device = page_table.device
        self.free_slots = torch.arange(num_pages, dtype=torch.int32, device=self.device) * page_size

    @property
    def free_pages(self) -> int:
        return int(self.free_slots.shape[0])

    def allocate_paged(self, reqs: Iterable) -> None:
        """Give every request the pages that its ``[cached_len, device_len)`` tokens start."""
        ps = self.page_size
        info: List[Tuple[int, int, int]] = []
        needed = 0
        for r in reqs:
            first, last = -(-r.cached_len // ps), -(-r.device_len // ps)
            if last > first:
                needed += last - first
                info.append((r.table_idx, first, last))
        if needed == 0:
            return
        if needed > self.free_pages:
            raise RuntimeError(f"out of KV pages: {needed} needed, {self.free_pages} free")
        pages, self.free_slots = self.free_slots[:needed], self.free_slots[needed:]
        tokens = (pages[:, None] + torch.arange(ps, dtype=torch.int32, device=self.device)).flatten()
        rows = torch.empty(needed * ps, dtype=torch.int64)
        cols = torch.empty(needed * ps, dtype=torch.int64)
        off = 0
        for table_idx, first, last in info:
            n = (last - first) * ps
            rows[off : off + n] = table_idx
            torch.arange(first * ps, last * ps, out=cols[off : off + n])
            off += n
        if self.device.type == "cuda":
            rows, cols = rows.pin_memory(), cols.pin_memory()
        self.page_table[rows.to(self.device, non_blocking=True), cols.to(self.device, non_blocking=True)] = tokens

    def out_loc(self, reqs: Iterable) -> torch.Tensor:
        """Token locations of every request's new positions, in batch order (the scheduler's
        ``out_loc``, python/minisgl/scheduler/scheduler.py:210)."""
        return torch.cat([self.page_table[r.table_idx, r.cached_len : r.device_len] for r in reqs])

    def free(self, table_idx: int, length: int) -> None:
        """Return the pages holding tokens ``[0, length)`` of a row (a finished request)."""
        if length > 0:
            self.free_slots = torch.cat((self.free_slots, self.page_table[table_idx, :length : self.page_size]))
