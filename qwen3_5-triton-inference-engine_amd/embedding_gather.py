"""Token embedding gather (MI355X HIP).

Drop-in for ``triton_kernels/embedding_gather.py``: op ``wy_lib::embedding_gather``
with the reference schema and assertions (:62-104) and
``call_embedding_gather_triton`` (:117-121).
"""

from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op("wy_lib::embedding_gather", mutates_args=(), device_types="cuda")
def embedding_gather(input_ids: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``weight[input_ids]``: input_ids ``[T]`` int32/int64, weight ``[V, D]`` bf16
    -> ``[T, D]`` bf16."""
    assert input_ids.ndim == 1
    assert input_ids.dtype in (torch.int32, torch.int64)
    assert input_ids.is_contiguous()
    assert weight.ndim == 2 and weight.dtype == torch.bfloat16
    assert weight.is_contiguous()
    assert input_ids.device == weight.device
    token_num = input_ids.shape[0]
    d_model = weight.shape[1]
    assert token_num > 0 and weight.shape[0] > 0
    assert d_model & (d_model - 1) == 0
    out = torch.empty((token_num, d_model), dtype=weight.dtype, device=weight.device)
    _lib.call("wy_embedding_gather", _lib.ptr(input_ids), int(input_ids.dtype == torch.int64),
              _lib.ptr(weight), weight.stride(0), weight.shape[0], _lib.ptr(out), out.stride(0), token_num,
              d_model, _lib.stream(weight.device))
    return out


@embedding_gather.register_fake
def _embedding_gather_fake(input_ids, weight):
    return weight.new_empty((input_ids.shape[0], weight.shape[1]))


def call_embedding_gather_triton(input_ids, weight):
    return embedding_gather(input_ids, weight)
