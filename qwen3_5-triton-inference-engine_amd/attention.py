"""Caller glue of the full-attention hot path: the op sequence the reference
runner issues around attention, from the normalised projections to the
gated ``o_proj`` input (engine/runner.py:313-398 prefill, :444-518 decode).

The projections (``gemm_2d``), q/k RMSNorm and ``o_proj`` sit outside this
path; callers pass their outputs in.  Views and strides are the ones the
reference builds, so the ops see the same layouts:

* prefill: q/k ``[T, H, D]`` -> ``[1, H, T, D]`` permuted views into
  ``partial_rope``; contiguous ``[total, H, D]`` copies into the varlen
  attention; ``ctx``/``gate`` as ``[1, H, T, D]`` views into the gate pack;
  ``k4[0]`` (strides ``(D, H*D, 1)``) into the page scatter.
* decode: ``pos.view(B, 1)`` int64 positions; ``[B, H, 1, D]`` into RoPE;
  ``[B, H, D]`` contiguous q/k/v into append + split + combine; ``[1, H, B, D]``
  into the gate pack (batch folded into tokens).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .attention_gate_pack import attention_gate_pack
from .gqa_attention_decode_paged import (
    call_paged_gqa_attention_decode_triton,
    paged_gqa_attention_decode_block,
    paged_gqa_attention_decode_fused,
    paged_kv_fill_varlen,
)
from .gqa_attention_varlen_causal import gqa_attention_varlen_causal
from .gqa_attention_varlen_causal import prefill_attention_block as _prefill_attention_block_op
from .partial_rope import partial_rope


@dataclass(frozen=True)
class PackedBatch:
    """Indices of B variable-length prompts packed into one flat sequence
    (reference engine/runner.py:73-124)."""

    cu_seqlens: torch.Tensor    # [B+1] int32
    seq_start: torch.Tensor     # [total] int32
    position_ids: torch.Tensor  # [1, total] int32, restarting at 0 per sequence
    max_seqlen: int
    lengths: tuple[int, ...]
    offsets: tuple[int, ...]    # host copy of cu_seqlens

    @property
    def batch(self) -> int:
        return len(self.lengths)

    @property
    def total_tokens(self) -> int:
        return self.offsets[-1]

    def slice_of(self, seq: int) -> slice:
        return slice(self.offsets[seq], self.offsets[seq + 1])


def build_packed_batch(lengths: list[int], *, device="cuda") -> PackedBatch:
    """Reference engine/runner.py:127-148."""
    offsets = [0]
    for n in lengths:
        offsets.append(offsets[-1] + n)
    total = offsets[-1]
    cu = torch.tensor(offsets, dtype=torch.int32, device=device)
    lens_t = torch.tensor(lengths, device=device)
    seq_start = torch.repeat_interleave(cu[:-1], lens_t)
    position_ids = (torch.arange(total, dtype=torch.int32, device=device)
                    - seq_start).unsqueeze(0)
    return PackedBatch(
        cu_seqlens=cu,
        seq_start=seq_start.to(torch.int32),
        position_ids=position_ids,
        max_seqlen=max(lengths),
        lengths=tuple(lengths),
        offsets=tuple(offsets),
    )


def prefill_attention_packed(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    gate: torch.Tensor,
    inv_freq: torch.Tensor,
    rotary_dim: int,
    packed: PackedBatch,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    trace: dict | None = None,
) -> torch.Tensor:
    """Packed prefill of one attention layer.

    q ``[T, Hq, D]`` and k ``[T, Hkv, D]`` (after q/k norm), v ``[T, Hkv*D]``
    or ``[T, Hkv, D]``, gate ``[T, Hq*D]``; returns the ``[T, Hq*D]`` input of
    ``o_proj`` and scatters the roped K and V into the page pools.
    """
    token_num, nh, d = q.shape
    nkv = k.shape[1]
    pos = packed.position_ids
    q4 = partial_rope(q.unsqueeze(0).permute(0, 2, 1, 3), pos, inv_freq, rotary_dim)
    k4 = partial_rope(k.unsqueeze(0).permute(0, 2, 1, 3), pos, inv_freq, rotary_dim)
    v4 = v.reshape(token_num, nkv, d).unsqueeze(0).permute(0, 2, 1, 3)
    ctx = gqa_attention_varlen_causal(
        q4[0].permute(1, 0, 2).contiguous(),
        k4[0].permute(1, 0, 2).contiguous(),
        v4[0].permute(1, 0, 2).contiguous(),
        packed.cu_seqlens,
        packed.max_seqlen,
    ).permute(1, 0, 2).unsqueeze(0)
    gate4 = gate.view(1, token_num, nh, d).permute(0, 2, 1, 3)
    gated = attention_gate_pack(ctx, gate4)
    paged_kv_fill_varlen(k_cache, v_cache, k4[0], v4[0], block_table,
                         packed.cu_seqlens, packed.max_seqlen)
    if trace is not None:
        trace["rope_q"], trace["rope_k"], trace["ctx"], trace["packed"] = q4, k4, ctx, gated
    return gated


def prefill_attention_block(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    gate: torch.Tensor,
    inv_freq: torch.Tensor,
    rotary_dim: int,
    packed: PackedBatch,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
) -> torch.Tensor:
    """``prefill_attention_packed`` in two launches (``wy_lib::prefill_attention_block``),
    bit-identical: same arguments, same ``[T, Hq*D]`` result and page contents.
    Rotary widths other than 64 take the op sequence."""
    token_num, nh, d = q.shape
    nkv = k.shape[1]
    if rotary_dim != 64:
        return prefill_attention_packed(q, k, v, gate, inv_freq, rotary_dim, packed, k_cache,
                                        v_cache, block_table)
    return _prefill_attention_block_op(
        q, k, v.reshape(token_num, nkv, d), gate.view(token_num, nh, d), packed.position_ids,
        inv_freq, rotary_dim, k_cache, v_cache, block_table, packed.cu_seqlens,
        packed.max_seqlen)


def decode_attention_step(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    gate: torch.Tensor,
    inv_freq: torch.Tensor,
    rotary_dim: int,
    pos: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    scratch,
) -> torch.Tensor:
    """One decode step of one attention layer for B sequences.

    q ``[B, Hq, D]``, k ``[B, Hkv, D]`` (after q/k norm, any strides), v
    ``[B, Hkv*D]``, gate ``[B, Hq*D]``; returns the ``[B, Hq*D]`` ``o_proj``
    input.  Appends the roped K and V at ``pos`` (caller advances ``pos``).
    Graph-capturable: nothing reads device values on the host.
    """
    batch, nh, d = q.shape
    nkv = k.shape[1]
    pos_ids = pos.view(batch, 1)
    q4 = partial_rope(q.unsqueeze(2), pos_ids, inv_freq, rotary_dim)
    k4 = partial_rope(k.unsqueeze(2), pos_ids, inv_freq, rotary_dim)
    q_new = q4[:, :, 0, :].contiguous()
    k_new = k4[:, :, 0, :].contiguous()
    v_new = v.reshape(batch, nkv, d).contiguous()
    counters = getattr(scratch, "counters", None)
    if counters is not None:
        # one launch: append + split + merge + gate
        m, l, acc = scratch
        out = paged_gqa_attention_decode_fused(
            q_new, k_new, v_new, k_cache, v_cache, block_table, pos, m, l, acc, counters,
            gate.view(batch, nh, d))
        return out.view(batch, nh * d)
    ctx = call_paged_gqa_attention_decode_triton(
        q_new, k_new, v_new, k_cache, v_cache, block_table, pos, scratch
    )
    gate4 = gate.reshape(batch, nh, d).permute(1, 0, 2).unsqueeze(0).contiguous()
    ctx4 = ctx.permute(1, 0, 2).unsqueeze(0).contiguous()
    return attention_gate_pack(ctx4, gate4)


def decode_attention_block(
    fused: torch.Tensor,
    q_norm: torch.Tensor,
    k_norm: torch.Tensor,
    eps: float,
    inv_freq: torch.Tensor,
    rotary_dim: int,
    pos: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    scratch,
    num_heads: int = 8,
    num_kv_heads: int = 2,
    head_dim: int = 256,
) -> torch.Tensor:
    """The decode attention of one layer from the fused q/gate/k/v projection
    output ``fused [B, 2*Hq*D + 2*Hkv*D]`` (engine/runner.py:462-517) to the
    ``[B, Hq*D]`` o_proj input, in one launch: the slices are passed as
    strided views, no copies.  ``scratch`` must carry merge counters
    (``allocate_split_scratch``)."""
    batch = fused.shape[0]
    qd, kd = num_heads * head_dim, num_kv_heads * head_dim
    q_raw = fused[:, :qd].view(batch, num_heads, head_dim)
    gate = fused[:, qd:2 * qd].view(batch, num_heads, head_dim)
    k_raw = fused[:, 2 * qd:2 * qd + kd].view(batch, num_kv_heads, head_dim)
    v_raw = fused[:, 2 * qd + kd:2 * qd + 2 * kd].view(batch, num_kv_heads, head_dim)
    counters = getattr(scratch, "counters", None)
    assert counters is not None, "the attention block needs a scratch with merge counters"
    m, l, acc = scratch
    out = paged_gqa_attention_decode_block(
        q_raw, gate, k_raw, v_raw, q_norm, k_norm, eps, inv_freq, rotary_dim, k_cache,
        v_cache, block_table, pos, m, l, acc, counters)
    return out.view(batch, num_heads * head_dim)
