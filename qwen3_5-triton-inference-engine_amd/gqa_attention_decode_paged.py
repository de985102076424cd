"""Paged KV cache + split-K GQA decode attention on MI355X HIP kernels.

Drop-in for ``triton_kernels/gqa_attention_decode_paged.py`` of the reference
engine: same ``wy_lib::`` op names, schemas, argument meaning and assertions,
same module-level names (``PAGE_SIZE``, ``MAX_SPLITS``, allocators,
``physical_rows``, ``paged_kv_fill``, ``call_paged_gqa_attention_decode_triton``).

Layout (unchanged from the reference, gqa_attention_decode_paged.py:29-36)::

    k_cache / v_cache   [num_pages, H_kv, 16, D]  bf16, one pool shared by all sequences
    block_table         [B, max_pages]            int32, logical -> physical page
    pos                 [B]                       int64, tokens already cached
    q / k_new / v_new   [B, H, D]                 bf16

Split partition.  The reference splits every sequence into
``ceil(npg / ceil(npg/128))`` page-aligned chunks.  The HIP pair here uses
``pps = max(ceil(npg/128), min_pages_per_split(B))`` pages per split in both the
split and the combine op, so short contexts do not write one 4 KiB fp32
partial per 16-token page.  The one-launch step and attention block (which
merge their own splits) also raise the floor to 128 pages for tables of
>= 1024 pages.  The scratch tensors keep the reference shapes; their contents
are a private contract between the ops.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib

PAGE_SIZE = 16
MAX_SPLITS = 128

# Lower bound on pages per split shared by split and combine (see module doc).
# Small batches keep 4 pages (64 tokens) per split so a lone sequence still
# spreads over many workgroups; large batches already fill the GPU and gain
# more from fewer partials to merge (24 pages = 384 tokens: at B=32 with
# contexts up to 2048 tokens this keeps the active splits within one round of
# the 256 CUs, one per CU in the kernels' balanced workgroup order).  Both ops
# derive it from the batch size alone, a static shape, so the pair stays
# graph-safe.
MIN_PAGES_PER_SPLIT = 4
MIN_PAGES_PER_SPLIT_LARGE_BATCH = 24
LARGE_BATCH = 16


def min_pages_per_split(batch: int) -> int:
    return MIN_PAGES_PER_SPLIT_LARGE_BATCH if batch >= LARGE_BATCH else MIN_PAGES_PER_SPLIT


# The one-launch step and block merge their own splits (no combine op has to
# agree on the partition).  For batches up to 256 the kernel raises the floor
# itself from the batch's total length (about one work item per CU: 64 x 32k
# tokens gets 1024-page splits, while one long sequence among short ones
# still gets many short splits); beyond 256 sequences a table of >= 1024
# pages (16k tokens) raises the floor to 128 pages.
LONG_CONTEXT_PAGES = 1024
MIN_PAGES_PER_SPLIT_LONG = 128
BALANCED_MAX_BATCH = 256


def min_pages_per_split_fused(batch: int, max_pages: int) -> int:
    if max_pages >= LONG_CONTEXT_PAGES and batch > BALANCED_MAX_BATCH:
        return MIN_PAGES_PER_SPLIT_LONG
    return min_pages_per_split(batch)


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


# --------------------------------------------------------------------------- allocation

def allocate_paged_kv_cache(
    num_pages: int,
    num_kv_heads: int,
    head_dim: int,
    *,
    device: torch.device | str = "cuda",
) -> tuple[torch.Tensor, torch.Tensor]:
    """Zeroed ``[num_pages, H_kv, PAGE, D]`` bf16 K and V pools
    (reference gqa_attention_decode_paged.py:100-111)."""
    shape = (num_pages, num_kv_heads, PAGE_SIZE, head_dim)
    k = torch.zeros(shape, dtype=torch.bfloat16, device=device)
    v = torch.zeros(shape, dtype=torch.bfloat16, device=device)
    return k, v


class SplitScratch(tuple):
    """``(m, l, acc)`` as in the reference, plus ``counters``: the int32
    counters the one-launch decode step uses to elect the workgroups that
    merge the splits (``B * H_kv`` per-(sequence, KV head) counters and
    ``B * H_kv * 8`` merge-group counters; allocated as ``B * H_q * 4``).
    Counters start at zero and every step leaves them at zero.  Unpacks like
    the reference's 3-tuple."""

    def __new__(cls, m, l, acc, counters):
        obj = super().__new__(cls, (m, l, acc))
        obj.counters = counters
        return obj


def allocate_split_scratch(
    num_q_heads: int,
    head_dim: int,
    *,
    batch: int = 1,
    device: torch.device | str = "cuda",
):
    """Split-K workspace shared by all attention layers: m, l ``[B, H_q, 128]``
    and acc ``[B, H_q, 128, D]`` fp32 (reference :591-609), plus the merge
    counters of the fused step (``.counters``, ``[B * H_q * 4]`` int32 zeros)."""
    m = torch.zeros((batch, num_q_heads, MAX_SPLITS), dtype=torch.float32, device=device)
    l = torch.zeros((batch, num_q_heads, MAX_SPLITS), dtype=torch.float32, device=device)
    acc = torch.zeros(
        (batch, num_q_heads, MAX_SPLITS, head_dim), dtype=torch.float32, device=device
    )
    counters = torch.zeros((batch * num_q_heads * 4,), dtype=torch.int32, device=device)
    return SplitScratch(m, l, acc, counters)


def physical_rows(
    block_table: torch.Tensor,
    token_index: torch.Tensor,
    num_kv_heads: int,
) -> torch.Tensor:
    """Logical token index -> row of ``k_cache.view(-1, D)``, shape ``[T, H]``:
    ``row(t, h) = (block_table[t // 16] * H + h) * 16 + t % 16``
    (reference :127-144, engine/paging.py:23).  Index arithmetic only; the
    HIP kernels compute the same address from the pool strides."""
    logical_page = token_index // PAGE_SIZE
    slot = token_index % PAGE_SIZE
    phys = block_table.index_select(0, logical_page.to(torch.int32)).to(torch.int64)
    heads = torch.arange(num_kv_heads, device=block_table.device, dtype=torch.int64)
    return (phys[:, None] * num_kv_heads + heads[None, :]) * PAGE_SIZE + slot[:, None]


# --------------------------------------------------------------------------- append

@torch.library.custom_op(
    "wy_lib::paged_kv_append", mutates_args=("k_cache", "v_cache"), device_types="cuda"
)
def paged_kv_append(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    block_table: torch.Tensor,
    pos: torch.Tensor,
) -> None:
    """Write the new token's K/V at slot ``pos[b]`` of sequence b's page
    (reference :254-305).  Bit-exact copy, one launch for K and V."""
    batch, num_kv_heads, head_dim = k_new.shape
    assert k_cache.shape[1] == num_kv_heads and k_cache.shape[3] == head_dim
    assert k_cache.shape[2] == PAGE_SIZE
    assert v_cache.shape == k_cache.shape
    assert k_new.shape == v_new.shape
    assert k_cache.dtype == v_cache.dtype == torch.bfloat16
    assert k_new.dtype == v_new.dtype == torch.bfloat16
    assert block_table.dtype == torch.int32 and block_table.shape[0] == batch
    assert pos.dtype == torch.int64 and pos.shape == (batch,)
    assert head_dim & (head_dim - 1) == 0
    assert block_table.stride(1) == 1 and pos.is_contiguous()
    _lib.call(
        "wy_paged_kv_append",
        _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.strides(k_cache), _lib.strides(v_cache),
        _lib.ptr(k_new), _lib.ptr(v_new), _lib.strides(k_new), _lib.strides(v_new),
        _lib.ptr(block_table), block_table.stride(0), _lib.ptr(pos),
        batch, num_kv_heads, head_dim, _lib.stream(k_cache.device),
    )


@paged_kv_append.register_fake
def _paged_kv_append_fake(k_cache, v_cache, k_new, v_new, block_table, pos) -> None:
    return None


# ---------------------------------------------------------------------- varlen fill

@torch.library.custom_op(
    "wy_lib::paged_kv_fill_varlen", mutates_args=("k_cache", "v_cache"), device_types="cuda"
)
def paged_kv_fill_varlen(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_packed: torch.Tensor,
    v_packed: torch.Tensor,
    block_table: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seqlen: int,
) -> None:
    """Scatter packed ``[H_kv, total, D]`` K/V (any strides) into each
    sequence's pages in one launch (reference :492-561).  Bit-exact; slots
    past a sequence's end and unreferenced pages stay untouched."""
    num_kv_heads, total_tokens, head_dim = k_packed.shape
    assert v_packed.shape == k_packed.shape
    assert k_cache.shape[1] == num_kv_heads and k_cache.shape[3] == head_dim
    assert k_cache.shape[2] == PAGE_SIZE
    assert v_cache.shape == k_cache.shape
    assert k_cache.dtype == v_cache.dtype == torch.bfloat16
    assert k_packed.dtype == v_packed.dtype == torch.bfloat16
    assert block_table.dtype == torch.int32 and block_table.ndim == 2
    assert cu_seqlens.dtype == torch.int32 and cu_seqlens.ndim == 1
    batch = cu_seqlens.shape[0] - 1
    assert block_table.shape[0] == batch, (
        f"block_table has {block_table.shape[0]} rows but cu_seqlens describes {batch} sequences"
    )
    assert block_table.shape[1] >= _cdiv(max_seqlen, PAGE_SIZE), (
        f"block_table rows hold {block_table.shape[1]} pages, too few for {max_seqlen} tokens"
    )
    assert head_dim & (head_dim - 1) == 0
    assert block_table.stride(1) == 1 and cu_seqlens.is_contiguous()
    _lib.call(
        "wy_paged_kv_fill_varlen",
        _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.strides(k_cache), _lib.strides(v_cache),
        _lib.ptr(k_packed), _lib.ptr(v_packed), _lib.strides(k_packed),
        _lib.strides(v_packed), _lib.ptr(block_table), block_table.stride(0),
        _lib.ptr(cu_seqlens), batch, num_kv_heads, head_dim, max_seqlen,
        _lib.stream(k_cache.device),
    )


@paged_kv_fill_varlen.register_fake
def _paged_kv_fill_varlen_fake(
    k_cache, v_cache, k_packed, v_packed, block_table, cu_seqlens, max_seqlen
) -> None:
    return None


def paged_kv_fill(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_prefill: torch.Tensor,
    v_prefill: torch.Tensor,
    block_table: torch.Tensor,
) -> None:
    """Single-sequence prefill scatter of ``[H, T, D]`` K/V through one
    block-table row (reference :355-375).  Runs the varlen HIP kernel with
    ``cu_seqlens = [0, T]``."""
    num_kv_heads, token_num, head_dim = k_prefill.shape
    assert v_prefill.shape == k_prefill.shape
    bt = block_table.reshape(1, -1)
    cu = torch.tensor([0, token_num], dtype=torch.int32, device=k_cache.device)
    paged_kv_fill_varlen(k_cache, v_cache, k_prefill, v_prefill, bt, cu, token_num)


# --------------------------------------------------------------------------- split

@torch.library.custom_op(
    "wy_lib::paged_gqa_attention_decode_split",
    mutates_args=("m_partial", "l_partial", "acc_partial"),
    device_types="cuda",
)
def paged_gqa_attention_decode_split(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    m_partial: torch.Tensor,
    l_partial: torch.Tensor,
    acc_partial: torch.Tensor,
    pos: torch.Tensor,
    seq_bucket: int,
) -> None:
    """Partial pass of split-K paged decode (reference :822-891).  Grid is a
    function of shapes only; ``pos``/``block_table`` are read on the device,
    so the op is graph-capturable.  ``seq_bucket`` was an autotune key in the
    reference and is accepted and ignored."""
    batch, num_q_heads, head_dim = q.shape
    num_pages, num_kv_heads, page, cache_dim = k_cache.shape
    assert page == PAGE_SIZE and cache_dim == head_dim
    assert v_cache.shape == k_cache.shape
    assert q.dtype == torch.bfloat16 and k_cache.dtype == torch.bfloat16
    assert block_table.dtype == torch.int32 and block_table.shape[0] == batch
    assert m_partial.shape == (batch, num_q_heads, MAX_SPLITS)
    assert acc_partial.shape == (batch, num_q_heads, MAX_SPLITS, head_dim)
    assert pos.dtype == torch.int64 and pos.shape == (batch,)
    assert num_q_heads % num_kv_heads == 0
    assert l_partial.shape == m_partial.shape and l_partial.stride() == m_partial.stride()
    assert m_partial.dtype == l_partial.dtype == acc_partial.dtype == torch.float32
    assert block_table.stride(1) == 1 and pos.is_contiguous()
    _lib.call(
        "wy_paged_decode_split",
        _lib.ptr(q), _lib.strides(q), _lib.ptr(k_cache), _lib.ptr(v_cache),
        _lib.strides(k_cache), _lib.strides(v_cache), _lib.ptr(block_table),
        block_table.stride(0), _lib.ptr(pos), _lib.ptr(m_partial), _lib.ptr(l_partial),
        _lib.ptr(acc_partial), _lib.strides(m_partial), _lib.strides(acc_partial),
        batch, num_q_heads, num_kv_heads, head_dim, block_table.shape[1],
        min_pages_per_split(batch), _lib.stream(q.device),
    )


@paged_gqa_attention_decode_split.register_fake
def _paged_split_fake(
    q, k_cache, v_cache, block_table, m_partial, l_partial, acc_partial, pos, seq_bucket
) -> None:
    return None


@torch.library.custom_op(
    "wy_lib::paged_gqa_attention_decode_combine", mutates_args=(), device_types="cuda"
)
def paged_gqa_attention_decode_combine(
    m_partial: torch.Tensor,
    l_partial: torch.Tensor,
    acc_partial: torch.Tensor,
    pos: torch.Tensor,
) -> torch.Tensor:
    """Merge the active splits into ``[B, H_q, D]`` bf16 (reference :901-939)."""
    batch, num_q_heads, _, head_dim = acc_partial.shape
    assert l_partial.stride() == m_partial.stride()
    assert pos.dtype == torch.int64 and pos.shape == (batch,) and pos.is_contiguous()
    out = torch.empty(
        (batch, num_q_heads, head_dim), dtype=torch.bfloat16, device=acc_partial.device
    )
    _lib.call(
        "wy_paged_decode_combine",
        _lib.ptr(m_partial), _lib.ptr(l_partial), _lib.ptr(acc_partial),
        _lib.strides(m_partial), _lib.strides(acc_partial), _lib.ptr(pos), _lib.ptr(out),
        _lib.strides(out), batch, num_q_heads, head_dim, min_pages_per_split(batch),
        _lib.stream(acc_partial.device),
    )
    return out


@paged_gqa_attention_decode_combine.register_fake
def _paged_combine_fake(m_partial, l_partial, acc_partial, pos) -> torch.Tensor:
    batch, num_q_heads, _, head_dim = acc_partial.shape
    return torch.empty(
        (batch, num_q_heads, head_dim), dtype=torch.bfloat16, device=acc_partial.device
    )


@torch.library.custom_op(
    "wy_lib::paged_gqa_attention_decode_fused",
    mutates_args=("k_cache", "v_cache", "m_partial", "l_partial", "acc_partial", "counters"),
    device_types="cuda",
)
def paged_gqa_attention_decode_fused(
    q: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    pos: torch.Tensor,
    m_partial: torch.Tensor,
    l_partial: torch.Tensor,
    acc_partial: torch.Tensor,
    counters: torch.Tensor,
    gate: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """append + split + combine (+ gate) in one launch; returns ``[B, H_q, D]``
    bf16.  Same result as the three reference ops in sequence (and, with
    ``gate``, followed by ``attention_gate_pack``): identical device code for
    the attention math and the same two bf16 roundings.  ``gate`` is
    ``[B, H_q, D]`` (any strides)."""
    batch, num_q_heads, head_dim = q.shape
    num_pages, num_kv_heads, page, cache_dim = k_cache.shape
    assert page == PAGE_SIZE and cache_dim == head_dim
    assert v_cache.shape == k_cache.shape
    assert k_new.shape == v_new.shape == (batch, num_kv_heads, head_dim)
    assert q.dtype == k_new.dtype == v_new.dtype == k_cache.dtype == v_cache.dtype == torch.bfloat16
    assert block_table.dtype == torch.int32 and block_table.shape[0] == batch
    assert block_table.stride(1) == 1
    assert pos.dtype == torch.int64 and pos.shape == (batch,) and pos.is_contiguous()
    assert m_partial.shape == (batch, num_q_heads, MAX_SPLITS)
    assert l_partial.shape == m_partial.shape and l_partial.stride() == m_partial.stride()
    assert acc_partial.shape == (batch, num_q_heads, MAX_SPLITS, head_dim)
    assert counters.dtype == torch.int32 and counters.is_contiguous()
    assert counters.numel() >= batch * num_kv_heads * 9
    assert num_q_heads % num_kv_heads == 0
    if gate is not None:
        assert gate.shape == q.shape and gate.dtype == torch.bfloat16
    out = torch.empty((batch, num_q_heads, head_dim), dtype=torch.bfloat16, device=q.device)
    _lib.call(
        "wy_paged_decode_step",
        _lib.ptr(q), _lib.strides(q), _lib.ptr(k_new), _lib.ptr(v_new), _lib.strides(k_new),
        _lib.strides(v_new), _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.strides(k_cache),
        _lib.strides(v_cache), _lib.ptr(block_table), block_table.stride(0), _lib.ptr(pos),
        _lib.ptr(m_partial), _lib.ptr(l_partial), _lib.ptr(acc_partial),
        _lib.strides(m_partial), _lib.strides(acc_partial), _lib.ptr(counters),
        _lib.ptr(gate), _lib.strides(gate), _lib.ptr(out), _lib.strides(out),
        batch, num_q_heads, num_kv_heads, head_dim, block_table.shape[1],
        min_pages_per_split_fused(batch, block_table.shape[1]), _lib.stream(q.device),
    )
    return out


@paged_gqa_attention_decode_fused.register_fake
def _paged_fused_fake(q, k_new, v_new, k_cache, v_cache, block_table, pos, m_partial,
                      l_partial, acc_partial, counters, gate=None) -> torch.Tensor:
    return torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)


@torch.library.custom_op(
    "wy_lib::paged_gqa_attention_decode_block",
    mutates_args=("k_cache", "v_cache", "m_partial", "l_partial", "acc_partial", "counters"),
    device_types="cuda",
)
def paged_gqa_attention_decode_block(
    q_raw: torch.Tensor,
    gate: torch.Tensor,
    k_raw: torch.Tensor,
    v_raw: torch.Tensor,
    q_norm: torch.Tensor,
    k_norm: torch.Tensor,
    eps: float,
    inv_freq: torch.Tensor,
    rotary_dim: int,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    pos: torch.Tensor,
    m_partial: torch.Tensor,
    l_partial: torch.Tensor,
    acc_partial: torch.Tensor,
    counters: torch.Tensor,
) -> torch.Tensor:
    """The decode attention block of one layer in one launch (the sequence of
    engine/runner.py:476-517 from the projection slices to the o_proj input):
    q/k RMSNorm (weight ``1 + w``), partial RoPE at ``pos``, K/V append,
    split-K attention + merge, sigmoid gate.  q_raw / gate ``[B, H_q, D]``,
    k_raw / v_raw ``[B, H_kv, D]``, any row strides.  Returns ``[B, H_q, D]``
    bf16, bit-identical to qwen_rmsnorm -> partial_rope ->
    paged_gqa_attention_decode_fused."""
    batch, num_q_heads, head_dim = q_raw.shape
    num_pages, num_kv_heads, page, cache_dim = k_cache.shape
    assert page == PAGE_SIZE and cache_dim == head_dim
    assert v_cache.shape == k_cache.shape
    assert gate.shape == q_raw.shape
    assert k_raw.shape == v_raw.shape == (batch, num_kv_heads, head_dim)
    for t in (q_raw, gate, k_raw, v_raw, q_norm, k_norm, k_cache, v_cache):
        assert t.dtype == torch.bfloat16
    assert q_raw.stride(-1) == 1 and k_raw.stride(-1) == 1 and v_raw.stride(-1) == 1
    assert q_norm.shape == k_norm.shape == (head_dim,)
    assert q_norm.is_contiguous() and k_norm.is_contiguous()
    assert inv_freq.dtype == torch.float32 and inv_freq.is_contiguous()
    assert inv_freq.numel() == rotary_dim // 2
    assert block_table.dtype == torch.int32 and block_table.shape[0] == batch
    assert block_table.stride(1) == 1
    assert pos.dtype == torch.int64 and pos.shape == (batch,) and pos.is_contiguous()
    assert m_partial.shape == (batch, num_q_heads, MAX_SPLITS)
    assert l_partial.shape == m_partial.shape and l_partial.stride() == m_partial.stride()
    assert acc_partial.shape == (batch, num_q_heads, MAX_SPLITS, head_dim)
    assert counters.dtype == torch.int32 and counters.is_contiguous()
    assert counters.numel() >= batch * num_kv_heads * 9
    out = torch.empty((batch, num_q_heads, head_dim), dtype=torch.bfloat16, device=q_raw.device)
    _lib.call(
        "wy_paged_decode_block",
        _lib.ptr(q_raw), _lib.strides(q_raw), _lib.ptr(gate), _lib.strides(gate),
        _lib.ptr(k_raw), _lib.strides(k_raw), _lib.ptr(v_raw), _lib.strides(v_raw),
        _lib.ptr(q_norm), _lib.ptr(k_norm), float(eps), _lib.ptr(inv_freq), rotary_dim,
        _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.strides(k_cache), _lib.strides(v_cache),
        _lib.ptr(block_table), block_table.stride(0), _lib.ptr(pos),
        _lib.ptr(m_partial), _lib.ptr(l_partial), _lib.ptr(acc_partial),
        _lib.strides(m_partial), _lib.strides(acc_partial), _lib.ptr(counters),
        _lib.ptr(out), _lib.strides(out), batch, num_q_heads, num_kv_heads, head_dim,
        block_table.shape[1], min_pages_per_split_fused(batch, block_table.shape[1]),
        _lib.stream(q_raw.device),
    )
    return out


@paged_gqa_attention_decode_block.register_fake
def _paged_block_fake(q_raw, gate, k_raw, v_raw, q_norm, k_norm, eps, inv_freq, rotary_dim,
                      k_cache, v_cache, block_table, pos, m_partial, l_partial, acc_partial,
                      counters) -> torch.Tensor:
    return torch.empty(q_raw.shape, dtype=torch.bfloat16, device=q_raw.device)


def _seq_bucket(seq_len: int) -> int:
    """Kept for interface parity with the reference (:950); the HIP kernels
    have fixed launch configurations, so the bucket selects nothing."""
    if seq_len <= 64:
        return 64
    if seq_len <= 256:
        return 256
    if seq_len <= 1024:
        return 1024
    if seq_len <= 4096:
        return 4096
    return 4097


def call_paged_gqa_attention_decode_triton(
    q: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    pos: torch.Tensor,
    scratch: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
) -> torch.Tensor:
    """Append + split + combine; returns ``[B, H_q, D]`` bf16 (reference
    :963-994).  The name is kept so callers switch by import only.  With a
    scratch from ``allocate_split_scratch`` (it carries merge counters) the
    three steps run as one launch; a plain ``(m, l, acc)`` tuple takes the
    three-op path."""
    if scratch is None:
        scratch = allocate_split_scratch(
            q.shape[1], q.shape[2], batch=q.shape[0], device=q.device
        )
    m_partial, l_partial, acc_partial = scratch
    counters = getattr(scratch, "counters", None)
    if counters is not None and _fused_ok(k_new, v_new):
        return paged_gqa_attention_decode_fused(
            q, k_new, v_new, k_cache, v_cache, block_table, pos, m_partial, l_partial,
            acc_partial, counters)
    paged_kv_append(k_cache, v_cache, k_new, v_new, block_table, pos)
    hint = k_cache.shape[0] * PAGE_SIZE
    paged_gqa_attention_decode_split(
        q, k_cache, v_cache, block_table, m_partial, l_partial, acc_partial, pos, hint
    )
    return paged_gqa_attention_decode_combine(m_partial, l_partial, acc_partial, pos)


def _fused_ok(k_new: torch.Tensor, v_new: torch.Tensor) -> bool:
    """The one-launch step reads k_new/v_new rows as 16-byte chunks."""
    return all(t.stride(2) == 1 and t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0
               and t.data_ptr() % 16 == 0 for t in (k_new, v_new))


paged_gqa_attention_decode = call_paged_gqa_attention_decode_triton


def page_stream_read(k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
                     pos: torch.Tensor) -> torch.Tensor:
    """Measurement helper, no counterpart in the reference: read every K/V page
    row a decode step at ``pos`` attends, once, with no attention math
    (``wy_page_stream_read``); returns the per-wavefront fp32 sums.  Its time
    is the HBM floor of the decode step's access pattern."""
    batch = pos.shape[0]
    num_kv_heads = k_cache.shape[1]
    assert k_cache.shape == v_cache.shape and k_cache.dtype == torch.bfloat16
    assert block_table.dtype == torch.int32 and block_table.stride(1) == 1
    assert pos.dtype == torch.int64 and pos.is_contiguous()
    lib = _lib.load()
    sums = torch.empty(lib.wy_page_stream_read_waves(), dtype=torch.float32,
                       device=k_cache.device)
    _lib.call("wy_page_stream_read", _lib.ptr(k_cache), _lib.ptr(v_cache),
              _lib.strides(k_cache), _lib.strides(v_cache), _lib.ptr(block_table),
              block_table.stride(0), _lib.ptr(pos), batch, num_kv_heads, k_cache.shape[3],
              _lib.ptr(sums), _lib.stream(k_cache.device))
    return sums
