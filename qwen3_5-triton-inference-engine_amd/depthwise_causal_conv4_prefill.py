"""Depthwise causal conv4 + SiLU over a prompt (MI355X HIP).

Drop-in for ``triton_kernels/depthwise_causal_conv4_prefill.py``: same op name
``wy_lib::depthwise_causal_conv4_prefill``, schema, assertions and output
(reference :104-176), ``call_depthwise_causal_conv4_prefill_triton`` (:187-192)
and ``build_seq_start`` (:195-206).
"""

from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op("wy_lib::depthwise_causal_conv4_prefill", mutates_args=(),
                         device_types="cuda")
def depthwise_causal_conv4_prefill(
    x: torch.Tensor,
    weight: torch.Tensor,
    seq_start: torch.Tensor | None = None,
) -> torch.Tensor:
    """x ``[T, D]`` bf16, weight ``[D, 4]`` or ``[D, 1, 4]`` bf16.  With
    ``seq_start`` (``[T]`` int32, each token's sequence start) token t never
    looks back past ``seq_start[t]``; without it the lower bound is 0."""
    assert x.ndim == 2
    assert weight.ndim in (2, 3)
    assert x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
    assert x.device == weight.device
    token_num, hidden_dim = x.shape
    assert token_num > 0 and hidden_dim > 0
    if weight.ndim == 2:
        assert weight.shape == (hidden_dim, 4)
        w_c, w_k = weight.stride(0), weight.stride(1)
    else:
        assert weight.shape == (hidden_dim, 1, 4)
        w_c, w_k = weight.stride(0), weight.stride(2)
    if seq_start is not None:
        assert seq_start.dtype == torch.int32 and seq_start.shape == (token_num,), (
            f"seq_start must be int32 [T]={(token_num,)}, got "
            f"{tuple(seq_start.shape)} {seq_start.dtype}"
        )
        assert seq_start.device == x.device
        seq_start = seq_start.contiguous()
    out = torch.empty_like(x)
    _lib.call(
        "wy_depthwise_causal_conv4_prefill", _lib.ptr(x), _lib.strides(x), _lib.ptr(weight),
        w_c, w_k, _lib.ptr(out), _lib.strides(out), _lib.ptr(seq_start), token_num, hidden_dim,
        _lib.stream(x.device),
    )
    return out


@depthwise_causal_conv4_prefill.register_fake
def _depthwise_causal_conv4_prefill_fake(x, weight, seq_start=None):
    return torch.empty_like(x)


def call_depthwise_causal_conv4_prefill_triton(x, weight, seq_start=None):
    return depthwise_causal_conv4_prefill(x, weight, seq_start)


def build_seq_start(lengths: list[int], *, device: torch.device | str = "cuda") -> torch.Tensor:
    """Lengths -> ``[total_tokens]`` int32: each token's sequence start."""
    starts, acc = [], 0
    for n in lengths:
        starts.append(acc)
        acc += n
    return torch.repeat_interleave(
        torch.tensor(starts, dtype=torch.int32, device=device),
        torch.tensor(lengths, device=device),
    )
