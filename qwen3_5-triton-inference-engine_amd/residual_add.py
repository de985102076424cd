"""Residual add (MI355X HIP).

Drop-in for ``triton_kernels/residual_add.py``: op ``wy_lib::residual_add``
with the reference schema and assertions (:23-52) and
``call_residual_add_triton`` (:62-66).
"""

from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op("wy_lib::residual_add", mutates_args=(), device_types="cuda")
def residual_add(x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    """``bf16(x + residual)`` elementwise (contiguous bf16 tensors)."""
    assert x.shape == residual.shape
    assert x.dtype == torch.bfloat16 and residual.dtype == torch.bfloat16
    assert x.device == residual.device
    assert x.is_contiguous() and residual.is_contiguous()
    assert x.numel() > 0
    out = torch.empty_like(x)
    _lib.call("wy_residual_add", _lib.ptr(x), _lib.ptr(residual), _lib.ptr(out), x.numel(),
              _lib.stream(x.device))
    return out


@residual_add.register_fake
def _residual_add_fake(x, residual):
    return torch.empty_like(x)


def call_residual_add_triton(x, residual):
    return residual_add(x, residual)
