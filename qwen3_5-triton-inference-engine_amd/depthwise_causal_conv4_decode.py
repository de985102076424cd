"""Depthwise causal conv4 decode step of the GDN mixer (MI355X HIP).

Drop-in for ``triton_kernels/depthwise_causal_conv4_decode.py``: same op name
``wy_lib::depthwise_causal_conv4_decode``, schema, assertions and layouts
(reference :152-205), plus ``call_depthwise_causal_conv4_decode_triton``
(:215-220) and ``conv_state_from_prefill`` (:222-235).
"""

from __future__ import annotations

import torch

from . import _lib

CONV_KERNEL_SIZE = 4


@torch.library.custom_op("wy_lib::depthwise_causal_conv4_decode", mutates_args=("state",),
                         device_types="cuda")
def depthwise_causal_conv4_decode(
    x: torch.Tensor,
    state: torch.Tensor,
    weight: torch.Tensor,
) -> torch.Tensor:
    """x ``[B, D]`` bf16 (one token per sequence); state ``[B, 4, D]`` bf16, the
    last four conv inputs, shifted in place; weight ``[4, D]`` bf16.  Returns
    ``silu(sum_r weight[r] * state'[r])`` as ``[B, D]`` bf16."""
    assert x.ndim == 2, "decode takes one token per sequence: x is [B,D]"
    assert state.ndim == 3 and weight.ndim == 2
    assert x.dtype == torch.bfloat16 and state.dtype == torch.bfloat16
    assert weight.dtype == torch.bfloat16
    assert x.device == state.device == weight.device
    batch, hidden_dim = x.shape
    assert state.shape == (batch, CONV_KERNEL_SIZE, hidden_dim), (
        f"state must be [B,4,D]={(batch, CONV_KERNEL_SIZE, hidden_dim)}, "
        f"got {tuple(state.shape)}"
    )
    assert weight.shape == (CONV_KERNEL_SIZE, hidden_dim), (
        f"weight must be [4,D]={(CONV_KERNEL_SIZE, hidden_dim)}, got {tuple(weight.shape)}"
    )
    assert state.is_contiguous() and weight.is_contiguous(), (
        "state/weight must be contiguous [B,4,D] / [4,D], not transposed [D,4] views"
    )
    out = torch.empty_like(x)
    _lib.call(
        "wy_depthwise_causal_conv4_decode", _lib.ptr(x), _lib.strides(x), _lib.ptr(state),
        _lib.strides(state), _lib.ptr(weight), _lib.strides(weight), _lib.ptr(out),
        _lib.strides(out), batch, hidden_dim, _lib.stream(x.device),
    )
    return out


@depthwise_causal_conv4_decode.register_fake
def _depthwise_causal_conv4_decode_fake(x, state, weight):
    return torch.empty_like(x)


def call_depthwise_causal_conv4_decode_triton(x, state, weight):
    return depthwise_causal_conv4_decode(x, state, weight)


def conv_state_from_prefill(x: torch.Tensor) -> torch.Tensor:
    """Prefill conv input ``[T, D]`` -> the decode conv state ``[4, D]``
    (contiguous): the last four rows, zero rows on top when T < 4."""
    token_num, hidden_dim = x.shape
    state = torch.zeros((CONV_KERNEL_SIZE, hidden_dim), dtype=x.dtype, device=x.device)
    take = min(token_num, CONV_KERNEL_SIZE)
    state[CONV_KERNEL_SIZE - take:] = x[-take:]
    return state


@torch.library.custom_op("wy_lib::conv_state_from_packed_prefill", mutates_args=("state",),
                         device_types="cuda")
def conv_state_from_packed_prefill(
    state: torch.Tensor,
    x: torch.Tensor,
    cu_seqlens: torch.Tensor,
) -> None:
    """Batched ``conv_state_from_prefill`` written straight into the cache:
    ``state[b]`` = the last four rows of sequence b in the packed ``x [T, D]``,
    zero rows on top for sequences shorter than four."""
    total_tokens, hidden_dim = x.shape
    batch = cu_seqlens.shape[0] - 1
    assert state.shape == (batch, CONV_KERNEL_SIZE, hidden_dim), (
        f"state {tuple(state.shape)} does not match (B={batch}, K={CONV_KERNEL_SIZE}, "
        f"D={hidden_dim})"
    )
    assert state.dtype == x.dtype
    assert cu_seqlens.dtype == torch.int32 and cu_seqlens.ndim == 1
    assert x.stride(1) == 1, "x must have a unit channel stride"
    assert state.stride(2) == 1
    _lib.call(
        "wy_conv_state_from_packed_prefill", _lib.ptr(state), _lib.strides(state), _lib.ptr(x),
        _lib.strides(x), _lib.ptr(cu_seqlens.contiguous()), batch, hidden_dim,
        _lib.stream(x.device),
    )


@conv_state_from_packed_prefill.register_fake
def _conv_state_from_packed_prefill_fake(state, x, cu_seqlens) -> None:
    return None
