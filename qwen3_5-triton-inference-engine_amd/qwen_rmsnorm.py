"""Qwen per-head RMSNorm with a ``(1 + w)`` weight (MI355X HIP).

Drop-in for ``triton_kernels/qwen_rmsnorm.py``: same op name
``wy_lib::qwen_rmsnorm``, schema, assertions and output layout (reference
:92-147), plus ``call_qwen_rmsnorm_triton`` (:158-163).  It is the q/k norm of
the decode attention block; ``wy_lib::paged_gqa_attention_decode_block``
applies the same device code inside its single launch.
"""

from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op("wy_lib::qwen_rmsnorm", mutates_args=(), device_types="cuda")
def qwen_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``bf16(x * rsqrt(mean(x^2) + eps) * (1 + weight))`` over the last dim,
    fp32 math.  x ``[B, M, D]`` with uniform strides (innermost 1) or any
    contiguous shape; the output is contiguous."""
    assert x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
    assert weight.is_contiguous()
    assert x.stride(-1) == 1
    d_model = x.shape[-1]
    assert d_model in (256, 1024)
    assert weight.shape == (d_model,)
    if x.ndim == 3:
        batch, rows = x.shape[0], x.shape[1]
        xs = (x.stride(0), x.stride(1), 1)
    else:
        assert x.is_contiguous(), "flattened rows need a contiguous input"
        batch, rows = 1, x.numel() // d_model
        xs = (0, d_model, 1)
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    os_ = (out.stride(0), out.stride(1), 1) if x.ndim == 3 else (0, d_model, 1)
    _lib.call(
        "wy_qwen_rmsnorm", _lib.ptr(x), _lib.i64_array(xs), _lib.ptr(weight), _lib.ptr(out),
        _lib.i64_array(os_), batch, rows, d_model, float(eps), _lib.stream(x.device),
    )
    return out


@qwen_rmsnorm.register_fake
def _qwen_rmsnorm_fake(x, weight, eps=1e-6) -> torch.Tensor:
    return torch.empty_like(x)


def call_qwen_rmsnorm_triton(x: torch.Tensor, weight: torch.Tensor,
                             eps: float = 1e-6) -> torch.Tensor:
    return qwen_rmsnorm(x, weight, eps)
