"""SwiGLU (MI355X HIP).

Drop-in for ``triton_kernels/swiglu.py``: op ``wy_lib::swiglu`` with the
reference schema and assertions (:72-111) and ``call_swiglu_triton`` (:120-124).
"""

from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op("wy_lib::swiglu", mutates_args=(), device_types="cuda")
def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``bf16(up * gate * sigmoid(gate))``; gate, up ``[M, N]`` bf16 (any
    strides, e.g. the two halves of the fused gate_up GEMV output)."""
    assert gate.ndim == 2 and up.ndim == 2
    assert gate.shape == up.shape
    assert gate.dtype == torch.bfloat16 and up.dtype == torch.bfloat16
    assert gate.device == up.device
    num_rows, num_cols = gate.shape
    assert num_rows > 0 and num_cols > 0
    out = torch.empty((num_rows, num_cols), dtype=gate.dtype, device=gate.device)
    _lib.call("wy_swiglu", _lib.ptr(gate), _lib.strides(gate), _lib.ptr(up), _lib.strides(up),
              _lib.ptr(out), num_rows, num_cols, _lib.stream(gate.device))
    return out


@swiglu.register_fake
def _swiglu_fake(gate, up):
    return gate.new_empty(gate.shape)


def call_swiglu_triton(gate, up):
    return swiglu(gate, up)
