"""Packed varlen causal GQA prefill attention on bf16 MFMA (MI355X HIP).

Drop-in for ``triton_kernels/gqa_attention_varlen_causal.py``: same op name
``wy_lib::gqa_attention_varlen_causal``, schema and assertions
(reference :214-278), plus ``build_cu_seqlens`` (:288).
"""

from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op(
    "wy_lib::gqa_attention_varlen_causal", mutates_args=(), device_types="cuda"
)
def gqa_attention_varlen_causal(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seqlen: int,
) -> torch.Tensor:
    """``out[t] = softmax_{j<=i}(q_i k_j^T / sqrt(D)) V`` within each packed
    sequence.  q/out ``[total, H_q, D]``, k/v ``[total, H_kv, D]`` bf16,
    ``cu_seqlens`` ``[B+1]`` int32, ``max_seqlen`` host int (grid size only)."""
    assert q.dtype == torch.bfloat16 and k.dtype == v.dtype == torch.bfloat16
    assert q.ndim == 3 and k.ndim == 3 and v.ndim == 3
    assert cu_seqlens.dtype == torch.int32 and cu_seqlens.ndim == 1

    total_tokens, num_q_head, d_model = q.shape
    assert k.shape == v.shape
    assert k.shape[0] == total_tokens and k.shape[2] == d_model
    num_kv_head = k.shape[1]
    assert num_q_head % num_kv_head == 0
    batch = cu_seqlens.numel() - 1
    assert batch >= 1
    assert cu_seqlens.is_contiguous()

    out = torch.empty_like(q)
    # Grids larger than the chip run as a persistent queue whose two ticket
    # counters live in a zeroed buffer kept per (device, stream); every launch
    # leaves them zero again.
    ws_bytes = _lib.load().wy_varlen_causal_prefill_workspace_bytes(
        batch, num_kv_head, max_seqlen
    )
    ws = _lib.stream_workspace(q.device, "prefill_queue", ws_bytes) if ws_bytes > 0 else None
    ws_bytes = ws.numel() if ws is not None else 0
    _lib.call(
        "wy_varlen_causal_prefill",
        _lib.ptr(q), _lib.strides(q), _lib.ptr(k), _lib.strides(k), _lib.ptr(v),
        _lib.strides(v), _lib.ptr(out), _lib.strides(out), _lib.ptr(cu_seqlens), batch,
        num_q_head, num_kv_head, d_model, max_seqlen, total_tokens, _lib.ptr(ws),
        ws_bytes, _lib.stream(q.device),
    )
    return out


@gqa_attention_varlen_causal.register_fake
def _gqa_attention_varlen_causal_fake(q, k, v, cu_seqlens, max_seqlen) -> torch.Tensor:
    return torch.empty_like(q)


@torch.library.custom_op(
    "wy_lib::prefill_attention_block",
    mutates_args=("k_cache", "v_cache"),
    device_types="cuda",
)
def prefill_attention_block(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    gate: torch.Tensor,
    position_ids: torch.Tensor,
    inv_freq: torch.Tensor,
    rotary_dim: int,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_table: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_seqlen: int,
) -> torch.Tensor:
    """The prefill attention sequence of the reference runner after the q/k
    norm (engine/runner.py:336-384) in two launches, bit-identical to it:
    partial RoPE of q and k, varlen causal attention, sigmoid gate pack, and
    the roped K / V scattered into the pages.  q ``[T, H_q, D]``, k / v
    ``[T, H_kv, D]``, gate ``[T, H_q, D]`` (views with a unit inner stride),
    ``position_ids`` ``[T]`` or ``[1, T]`` int32/int64, ``rotary_dim`` 64.
    Returns the ``[T, H_q * D]`` o_proj input."""
    assert q.dtype == k.dtype == v.dtype == gate.dtype == torch.bfloat16
    assert q.ndim == 3 and k.ndim == 3 and v.ndim == 3 and gate.shape == q.shape
    total_tokens, num_q_head, d_model = q.shape
    num_kv_head = k.shape[1]
    assert k.shape == v.shape and k.shape[0] == total_tokens and k.shape[2] == d_model
    if gate.stride(2) != 1 or gate.stride(0) % 8 or gate.stride(1) % 8 or gate.data_ptr() % 16:
        gate = gate.contiguous()   # the epilogue reads 16-byte pieces of gate rows
    assert cu_seqlens.dtype == torch.int32 and cu_seqlens.is_contiguous()
    assert position_ids.dtype in (torch.int32, torch.int64)
    assert position_ids.numel() == total_tokens
    assert inv_freq.dtype == torch.float32 and inv_freq.is_contiguous()
    batch = cu_seqlens.numel() - 1
    assert batch >= 1
    pos = position_ids.reshape(-1)
    k_roped = torch.empty((total_tokens, num_kv_head, d_model), dtype=q.dtype, device=q.device)
    rope_table = torch.empty((total_tokens, rotary_dim), dtype=torch.float32, device=q.device)
    out = torch.empty((total_tokens, num_q_head * d_model), dtype=q.dtype, device=q.device)
    ws_bytes = _lib.load().wy_varlen_causal_prefill_workspace_bytes(
        batch, num_kv_head, max_seqlen
    )
    ws = _lib.stream_workspace(q.device, "prefill_queue", ws_bytes) if ws_bytes > 0 else None
    _lib.call(
        "wy_prefill_attention_block",
        _lib.ptr(q), _lib.strides(q), _lib.ptr(k), _lib.strides(k), _lib.ptr(v),
        _lib.strides(v), _lib.ptr(gate), _lib.strides(gate), _lib.ptr(pos), pos.stride(0),
        int(pos.dtype == torch.int64), _lib.ptr(inv_freq), rotary_dim, _lib.ptr(k_cache),
        _lib.ptr(v_cache), _lib.strides(k_cache), _lib.strides(v_cache), _lib.ptr(block_table),
        block_table.stride(0), _lib.ptr(cu_seqlens), batch, num_q_head, num_kv_head, d_model,
        max_seqlen, total_tokens, _lib.ptr(k_roped), _lib.ptr(rope_table), _lib.ptr(out),
        _lib.ptr(ws),
        ws.numel() if ws is not None else 0, _lib.stream(q.device),
    )
    return out


@prefill_attention_block.register_fake
def _prefill_attention_block_fake(q, k, v, gate, position_ids, inv_freq, rotary_dim, k_cache,
                                  v_cache, block_table, cu_seqlens, max_seqlen):
    return q.new_empty((q.shape[0], q.shape[1] * q.shape[2]))


def build_cu_seqlens(
    lengths: list[int], *, device: torch.device | str = "cuda"
) -> tuple[torch.Tensor, int]:
    """Lengths -> (cu_seqlens [B+1] int32, max_seqlen) (reference :288)."""
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return (
        torch.tensor(cu, dtype=torch.int32, device=device),
        max(lengths) if lengths else 0,
    )
