"""Physical page allocation and the device block table.

Same contract as the reference's ``engine/paging.py``:

* host side: a free list of physical page ids (``PagePool``);
* device side: ``block_table`` ``[B, max_pages]`` int32, logical page -> physical
  page, one row per sequence.  Kernels read it when they run, so the host may
  write newly reserved pages between graph replays; its shape never changes.

Token t of sequence b lives at row ``(block_table[b, t // 16] * H + h) * 16 +
t % 16`` of ``k_cache.view(-1, D)``.
"""

from __future__ import annotations

import torch

from .gqa_attention_decode_paged import PAGE_SIZE


def allocate_block_table(
    max_pages: int, *, batch: int = 1, device: torch.device | str = "cuda"
) -> torch.Tensor:
    """Zeroed ``[B, max_pages]`` int32 table (reference engine/paging.py:55)."""
    return torch.zeros((batch, max_pages), dtype=torch.int32, device=device)


class PagePool:
    """Host free list of physical pages (reference engine/paging.py:71-103).

    ``alloc`` takes pages from the tail and ``free`` appends them back, so a
    repeated alloc/free cycle hands out the same page ids (reproducible runs).
    """

    def __init__(self, num_pages: int):
        assert num_pages > 0
        self.num_pages = num_pages
        self._free: list[int] = list(range(num_pages))

    @property
    def num_free(self) -> int:
        return len(self._free)

    def alloc(self, count: int) -> list[int]:
        assert count <= len(self._free), (
            f"out of pages: need {count}, {len(self._free)} free of {self.num_pages} "
            f"({PAGE_SIZE} tokens per page); raise num_pages or lower max_tokens"
        )
        if count == 0:
            return []
        taken = self._free[-count:]
        del self._free[-count:]
        return taken

    def free(self, pages: list[int]) -> None:
        self._free.extend(pages)

    def reset(self) -> None:
        self._free = list(range(self.num_pages))


class SequencePages:
    """Block table of a batch plus the host record of each row's pages
    (reference engine/paging.py:106-177)."""

    def __init__(self, max_pages: int, *, batch: int = 1,
                 device: torch.device | str = "cuda"):
        self.max_pages = max_pages
        self.batch = batch
        self.block_table = allocate_block_table(max_pages, batch=batch, device=device)
        self.pages: list[list[int]] = [[] for _ in range(batch)]

    def reserve(self, token_num: int, pool: PagePool, *, seq: int = 0) -> None:
        """Make sequence ``seq`` able to hold ``token_num`` tokens, taking only
        the missing pages from ``pool``.  Must run before any forward that
        writes those positions; kernels do no bounds checks."""
        need = (token_num + PAGE_SIZE - 1) // PAGE_SIZE
        assert need <= self.max_pages, (
            f"{token_num} tokens need {need} pages, block table holds {self.max_pages}"
        )
        held = self.pages[seq]
        if need <= len(held):
            return
        new_pages = pool.alloc(need - len(held))
        self.block_table[seq, len(held):need] = torch.tensor(
            new_pages, dtype=torch.int32, device=self.block_table.device
        )
        held.extend(new_pages)

    def reserve_all(self, token_num: int, pool: PagePool) -> None:
        for seq in range(self.batch):
            self.reserve(token_num, pool, seq=seq)

    def release(self, pool: PagePool, *, seq: int | None = None) -> None:
        """Return pages to the pool (all rows when ``seq`` is None) and zero the
        released block-table rows."""
        targets = range(self.batch) if seq is None else [seq]
        for b in targets:
            pool.free(self.pages[b])
            self.pages[b] = []
        if seq is None:
            self.block_table.zero_()
        else:
            self.block_table[seq].zero_()

    def capacity(self, seq: int = 0) -> int:
        return len(self.pages[seq]) * PAGE_SIZE
