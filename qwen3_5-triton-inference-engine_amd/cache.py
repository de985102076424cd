"""Attention-layer caches of a decode run (the full-attention part of the
reference's ``engine/cache.py:52-217``).

One page pool per attention layer (``[num_pages, H_kv, 16, D]`` bf16 K and V),
one block table shared by all layers, ``pos`` ``[B]`` int64 on the device and
one split-K scratch shared by all layers.  Sizing follows the reference:
``pages_per_seq = ceil(max_len / 16) + 1``, ``num_pages = pages_per_seq * B``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .gqa_attention_decode_paged import (
    PAGE_SIZE,
    allocate_paged_kv_cache,
    allocate_split_scratch,
)
from .paging import PagePool, SequencePages


@dataclass
class AttnCaches:
    pos: torch.Tensor                       # [B] int64
    k_caches: list[torch.Tensor]            # per attention layer
    v_caches: list[torch.Tensor]
    split_scratch: tuple[torch.Tensor, torch.Tensor, torch.Tensor]
    pages: SequencePages
    page_pool: PagePool
    max_len: int
    batch: int = 1

    @property
    def block_table(self) -> torch.Tensor:
        return self.pages.block_table

    def reserve(self, token_num: int) -> None:
        assert token_num <= self.max_len, (
            f"need room for {token_num} tokens, cache holds {self.max_len}"
        )
        self.pages.reserve_all(token_num, self.page_pool)

    def reset(self) -> None:
        """Zero positions, pools and scratch and return every page."""
        self.pos.zero_()
        for t in (*self.k_caches, *self.v_caches, *self.split_scratch):
            t.zero_()
        self.pages.release(self.page_pool)

    def memory_bytes(self) -> dict[str, int]:
        def total(ts):
            return sum(t.numel() * t.element_size() for t in ts)

        return {"kv": total(self.k_caches) + total(self.v_caches),
                "scratch": total(self.split_scratch)}


def allocate_attn_caches(
    num_layers: int,
    max_len: int,
    *,
    batch: int = 1,
    num_q_heads: int = 8,
    num_kv_heads: int = 2,
    head_dim: int = 256,
    device: torch.device | str = "cuda",
) -> AttnCaches:
    pages_per_seq = (max_len + PAGE_SIZE - 1) // PAGE_SIZE + 1
    num_pages = pages_per_seq * batch
    ks, vs = [], []
    for _ in range(num_layers):
        k, v = allocate_paged_kv_cache(num_pages, num_kv_heads, head_dim, device=device)
        ks.append(k)
        vs.append(v)
    return AttnCaches(
        pos=torch.zeros(batch, dtype=torch.int64, device=device),
        k_caches=ks,
        v_caches=vs,
        split_scratch=allocate_split_scratch(num_q_heads, head_dim, batch=batch,
                                             device=device),
        pages=SequencePages(pages_per_seq, batch=batch, device=device),
        page_pool=PagePool(num_pages),
        max_len=max_len,
        batch=batch,
    )
