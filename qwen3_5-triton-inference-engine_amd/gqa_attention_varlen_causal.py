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
