"""LM head fused with the vocabulary argmax (MI355X HIP).

Drop-in for ``triton_kernels/vocab_argmax.py``: op ``wy_lib::lm_head_argmax``
with the reference schema, assertions and return shapes (:137-224) and
``call_lm_head_argmax_triton`` (:236-240).  The 248320-wide logits are never
written: a persistent MFMA kernel streams the weight once and keeps the best
(logit, index) per row; a second launch folds the per-workgroup winners.
"""

from __future__ import annotations

import torch

from . import _lib

MAX_ROWS = 64


@torch.library.custom_op("wy_lib::lm_head_argmax", mutates_args=(), device_types="cuda")
def lm_head_argmax(hidden: torch.Tensor, weight: torch.Tensor,
                   last_only: bool = True) -> torch.Tensor:
    """``argmax(weight @ hidden[m])`` per row (first index on ties).
    ``last_only=True``: hidden ``[T, D]`` -> a 0-dim int64 for the last row
    (prefill); ``False``: hidden ``[B, D]`` -> ``[B]`` int64 (batched decode)."""
    assert hidden.ndim == 2 and weight.ndim == 2
    assert hidden.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
    assert hidden.device == weight.device
    assert hidden.is_contiguous() and weight.is_contiguous()
    token_num, hidden_size = hidden.shape
    vocab_size, weight_hidden_size = weight.shape
    assert token_num > 0 and vocab_size > 0
    assert weight_hidden_size == hidden_size
    assert hidden_size % 256 == 0
    rows_view = hidden[token_num - 1:] if last_only else hidden
    rows = rows_view.shape[0]
    assert rows <= MAX_ROWS, f"at most {MAX_ROWS} rows per call"
    lib = _lib.load()
    ws_bytes = lib.wy_lm_head_argmax_workspace_bytes(rows, hidden_size, vocab_size)
    ws = _lib.stream_workspace(hidden.device, "lm_head_argmax", ws_bytes)
    token_id = torch.empty((rows,), dtype=torch.int64, device=hidden.device)
    _lib.call("wy_lm_head_argmax", _lib.ptr(rows_view), rows_view.stride(0), _lib.ptr(weight),
              weight.stride(0), _lib.ptr(token_id), rows, hidden_size, vocab_size, _lib.ptr(ws),
              ws.numel(), _lib.stream(hidden.device))
    return token_id[0] if last_only else token_id


@lm_head_argmax.register_fake
def _lm_head_argmax_fake(hidden, weight, last_only=True):
    shape = () if last_only else (hidden.shape[0],)
    return torch.empty(shape, dtype=torch.int64, device=hidden.device)


def call_lm_head_argmax_triton(hidden, weight):
    return lm_head_argmax(hidden, weight)
