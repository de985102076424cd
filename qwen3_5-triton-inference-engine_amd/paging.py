"""Physical page allocation and the device block table.

Contract kept from the reference's ``engine/paging.py:55-177`` (callers and
existing caches depend on it):

* ``allocate_block_table`` -> zeroed ``[B, max_pages]`` int32 table, one row per
  sequence, logical page -> physical page.  Kernels read it when they run, so
  the host may write newly reserved pages between graph replays; its shape and
  address never change.
* ``PagePool.alloc`` hands out pages from the tail of the free order and
  ``free`` puts them back at the tail, so an alloc/free cycle returns the same
  page ids (reproducible runs); asking for more pages than are free raises
  ``AssertionError`` on the host.
* ``SequencePages.reserve`` takes only the pages a sequence is missing,
  ``release`` returns them and zeroes the released rows, ``capacity`` is the
  tokens the held pages cover.

Token t of sequence b lives at row ``(block_table[b, t // 16] * H + h) * 16 +
t % 16`` of ``k_cache.view(-1, D)``.

Design here: the pool is a fixed int32 stack with a top index (alloc/free are
slice copies, no per-page Python objects); a batch's page ownership is a host
mirror of the device table plus a held-page count per row, and a reservation
writes the row's new entries with one host->device copy of that slice.
"""

from __future__ import annotations

import numpy as np
import torch

from .gqa_attention_decode_paged import PAGE_SIZE


def allocate_block_table(
    max_pages: int, *, batch: int = 1, device: torch.device | str = "cuda"
) -> torch.Tensor:
    """Zeroed ``[batch, max_pages]`` int32 table (reference engine/paging.py:55)."""
    return torch.zeros((batch, max_pages), dtype=torch.int32, device=device)


class PagePool:
    """Free physical pages as a stack: ``_stack[:_top]`` are free, the next
    allocation takes ``_stack[_top - count:_top]`` (reference interface:
    engine/paging.py:71-103)."""

    def __init__(self, num_pages: int):
        assert num_pages > 0, f"a page pool needs at least one page (got {num_pages})"
        self.num_pages = num_pages
        self._stack = np.arange(num_pages, dtype=np.int32)
        self._top = num_pages

    @property
    def num_free(self) -> int:
        return self._top

    def alloc(self, count: int) -> list[int]:
        assert 0 <= count <= self._top, (
            f"page pool exhausted: {count} pages requested, {self._top} of "
            f"{self.num_pages} free ({PAGE_SIZE}-token pages)"
        )
        self._top -= count
        return self._stack[self._top:self._top + count].tolist()

    def free(self, pages) -> None:
        n = len(pages)
        assert self._top + n <= self.num_pages, "more pages freed than the pool holds"
        self._stack[self._top:self._top + n] = pages
        self._top += n

    def reset(self) -> None:
        self._stack[:] = np.arange(self.num_pages, dtype=np.int32)
        self._top = self.num_pages


class SequencePages:
    """Device block table of a batch plus the host record of which pages each
    row holds (reference interface: engine/paging.py:106-177)."""

    def __init__(self, max_pages: int, *, batch: int = 1,
                 device: torch.device | str = "cuda"):
        self.max_pages = max_pages
        self.batch = batch
        self.block_table = allocate_block_table(max_pages, batch=batch, device=device)
        self._rows = np.zeros((batch, max_pages), dtype=np.int32)   # host mirror
        self._held = np.zeros(batch, dtype=np.int64)                  # pages per row

    @property
    def pages(self) -> list[list[int]]:
        """Physical pages held by each sequence, in logical order."""
        return [self._rows[b, :self._held[b]].tolist() for b in range(self.batch)]

    def reserve(self, token_num: int, pool: PagePool, *, seq: int = 0) -> None:
        """Let sequence ``seq`` hold ``token_num`` tokens, taking only the missing
        pages from ``pool``.  Call it before any forward that writes those
        positions: the kernels do no bounds checks."""
        want = -(-token_num // PAGE_SIZE)
        assert want <= self.max_pages, (
            f"sequence {seq}: {token_num} tokens span {want} pages; the block table "
            f"has {self.max_pages} per sequence"
        )
        have = int(self._held[seq])
        if want <= have:
            return
        self._rows[seq, have:want] = pool.alloc(want - have)
        self._held[seq] = want
        self.block_table[seq, have:want].copy_(torch.from_numpy(self._rows[seq, have:want]))

    def reserve_all(self, token_num: int, pool: PagePool) -> None:
        for seq in range(self.batch):
            self.reserve(token_num, pool, seq=seq)

    def release(self, pool: PagePool, *, seq: int | None = None) -> None:
        """Give the pages of ``seq`` (every row when None) back to the pool, in
        row order, and zero the released block-table rows."""
        rows = range(self.batch) if seq is None else (seq,)
        for b in rows:
            pool.free(self._rows[b, :self._held[b]])
            self._rows[b] = 0
            self._held[b] = 0
        if seq is None:
            self.block_table.zero_()
        else:
            self.block_table[seq].zero_()

    def capacity(self, seq: int = 0) -> int:
        return int(self._held[seq]) * PAGE_SIZE
