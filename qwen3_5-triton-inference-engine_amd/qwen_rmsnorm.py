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


@torch.library.custom_op("wy_lib::add_rmsnorm", mutates_args=(), device_types="cuda")
def add_rmsnorm(h: torch.Tensor, x: torch.Tensor, weight: torch.Tensor,
                eps: float = 1e-6) -> tuple[torch.Tensor, torch.Tensor]:
    """``(s, qwen_rmsnorm(s))`` with ``s = bf16(h + x)``: a decoder layer's
    residual add and the RMSNorm after it in one launch, equal bit for bit to
    ``residual_add`` followed by ``qwen_rmsnorm``.  h, x contiguous
    ``[..., D]`` bf16."""
    assert h.shape == x.shape
    assert h.dtype == torch.bfloat16 and x.dtype == torch.bfloat16
    assert weight.dtype == torch.bfloat16 and weight.is_contiguous()
    assert h.is_contiguous() and x.is_contiguous()
    d_model = x.shape[-1]
    assert d_model % 256 == 0 and d_model <= 1024 and weight.shape == (d_model,)
    s = torch.empty_like(x)
    out = torch.empty_like(x)
    _lib.call("wy_add_rmsnorm", _lib.ptr(h), _lib.ptr(x), _lib.ptr(weight), _lib.ptr(s),
              _lib.ptr(out), x.numel() // d_model, d_model, float(eps), _lib.stream(x.device))
    return s, out


@add_rmsnorm.register_fake
def _add_rmsnorm_fake(h, x, weight, eps=1e-6):
    return torch.empty_like(x), torch.empty_like(x)


def call_qwen_rmsnorm_triton(x: torch.Tensor, weight: torch.Tensor,
                             eps: float = 1e-6) -> torch.Tensor:
    return qwen_rmsnorm(x, weight, eps)
