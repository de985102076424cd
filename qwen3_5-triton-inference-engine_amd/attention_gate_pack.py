"""Sigmoid output gate + head packing (MI355X HIP).

Drop-in for ``triton_kernels/attention_gate_pack.py``: op
``wy_lib::attention_gate_pack`` (:77-126).
``out[t, h*D + d] = bf16(x[0,h,t,d] * sigmoid(float(gate[0,h,t,d])))``;
x and gate are strided ``[1, H, T, D]`` views, out is ``[T, H*D]`` contiguous.
"""

from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op("wy_lib::attention_gate_pack", mutates_args=(), device_types="cuda")
def attention_gate_pack(x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    assert x.ndim == 4 and gate.ndim == 4
    assert x.shape == gate.shape
    assert x.dtype == torch.bfloat16 and gate.dtype == torch.bfloat16
    assert x.device == gate.device

    batch_size, num_heads, token_num, head_dim = x.shape
    assert batch_size == 1
    assert token_num > 0
    assert head_dim > 0 and head_dim & (head_dim - 1) == 0

    out = torch.empty((token_num, num_heads * head_dim), dtype=x.dtype, device=x.device)
    _lib.call(
        "wy_attention_gate_pack",
        _lib.ptr(x), _lib.strides(x), _lib.ptr(gate), _lib.strides(gate), _lib.ptr(out),
        num_heads, token_num, head_dim, _lib.stream(x.device),
    )
    return out


@attention_gate_pack.register_fake
def _attention_gate_pack_fake(x, gate) -> torch.Tensor:
    return torch.empty((x.shape[2], x.shape[1] * x.shape[3]), dtype=x.dtype, device=x.device)


def call_attention_gate_pack_triton(x, gate):
    """Name kept from the reference (attention_gate_pack.py:140)."""
    return attention_gate_pack(x, gate)
