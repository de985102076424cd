"""GDN gated RMSNorm (MI355X HIP).

Drop-in for ``triton_kernels/gdn_gated_rmsnorm.py``: same op name
``wy_lib::gdn_gated_rmsnorm``, schema, assertions and output (reference
:88-137), plus ``call_gdn_gated_rmsnorm_triton`` (:148-153).
"""

from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op("wy_lib::gdn_gated_rmsnorm", mutates_args=(), device_types="cuda")
def gdn_gated_rmsnorm(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``bf16(x * rsqrt(mean(x^2) + 1e-6) * weight * z * sigmoid(z))`` over the
    last dim; x, z ``[T, H, D]`` bf16, weight ``[D]`` fp32.  Output contiguous."""
    assert x.ndim == 3 and z.ndim == 3
    assert x.shape == z.shape
    assert x.dtype == torch.bfloat16 and z.dtype == torch.bfloat16
    assert weight.ndim == 1 and weight.dtype == torch.float32
    assert x.device == z.device == weight.device
    token_num, head_num, d_model = x.shape
    assert token_num > 0
    assert weight.shape == (d_model,)
    assert head_num & (head_num - 1) == 0
    assert d_model & (d_model - 1) == 0
    weight = weight.contiguous()
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    _lib.call(
        "wy_gdn_gated_rmsnorm", _lib.ptr(x), _lib.strides(x), _lib.ptr(z), _lib.strides(z),
        _lib.ptr(weight), _lib.ptr(out), token_num, head_num, d_model, _lib.stream(x.device),
    )
    return out


@gdn_gated_rmsnorm.register_fake
def _gdn_gated_rmsnorm_fake(x, z, weight):
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


def call_gdn_gated_rmsnorm_triton(x, z, weight):
    return gdn_gated_rmsnorm(x, z, weight)
