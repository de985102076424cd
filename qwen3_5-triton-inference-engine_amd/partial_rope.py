"""Partial rotate-half RoPE (MI355X HIP).

Drop-in for ``triton_kernels/partial_rope.py``: op ``wy_lib::partial_rope``
with the reference schema and assertions (:145-198).  Dims ``[0, R/2)`` and
``[R/2, R)`` rotate as a pair with fp32 ``cos/sin(float(pos) * inv_freq)``;
dims ``[R, D)`` are copied bit-exactly.  The output keeps x's strides
(``empty_like``), as in the reference.
"""

from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op("wy_lib::partial_rope", mutates_args=(), device_types="cuda")
def partial_rope(
    x: torch.Tensor,
    position_ids: torch.Tensor,
    inv_freq: torch.Tensor,
    rotary_dim: int,
) -> torch.Tensor:
    assert x.ndim == 4
    assert x.dtype == torch.bfloat16
    assert position_ids.ndim == 2
    assert position_ids.dtype in (torch.int32, torch.int64)
    assert inv_freq.ndim == 1 and inv_freq.dtype == torch.float32
    assert x.device == position_ids.device == inv_freq.device

    batch_size, num_heads, token_num, head_dim = x.shape
    assert position_ids.shape == (batch_size, token_num)
    assert rotary_dim > 0 and rotary_dim <= head_dim and rotary_dim % 2 == 0
    assert inv_freq.shape == (rotary_dim // 2,)
    assert inv_freq.is_contiguous()

    out = torch.empty_like(x)
    _lib.call(
        "wy_partial_rope",
        _lib.ptr(x), _lib.strides(x), _lib.ptr(out), _lib.strides(out),
        _lib.ptr(position_ids), _lib.strides(position_ids),
        int(position_ids.dtype == torch.int64), _lib.ptr(inv_freq), batch_size,
        num_heads, token_num, head_dim, rotary_dim, _lib.stream(x.device),
    )
    return out


@partial_rope.register_fake
def _partial_rope_fake(x, position_ids, inv_freq, rotary_dim) -> torch.Tensor:
    return torch.empty_like(x)


def call_partial_rope_triton(x, position_ids, inv_freq, rotary_dim):
    """Name kept from the reference (partial_rope.py:209)."""
    return partial_rope(x, position_ids, inv_freq, rotary_dim)


def rope_inv_freq(rotary_dim: int, theta: float, *, device="cuda") -> torch.Tensor:
    """``inv_freq[j] = 1 / theta^(2j/R)`` fp32, as built by the reference
    runner (engine/runner.py:181-190)."""
    return (
        1.0
        / (theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32, device=device)
                     / rotary_dim))
    ).contiguous()
