"""Gated DeltaNet delta-rule recurrence (MI355X HIP).

Drop-in for the recurrent ops of ``triton_kernels/gdn_recurrent_prefill.py``:
same op names ``wy_lib::gdn_recurrent_decode`` and
``wy_lib::gdn_recurrent_prefill_sequential``, schemas, assertions and
returned layouts (reference :1050-1146, :1185-1260), plus the
``call_*_triton`` wrappers (:1174-1182, :1274-1282).  Both run one launch of
``csrc/gdn.hip``; there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib


def _check_common(q, k, v, beta, g):
    # the reference's preconditions (gdn_recurrent_prefill.py:1070-1087, :1199-1211)
    assert q.ndim == 3 and k.ndim == 3 and v.ndim == 3
    assert q.shape == k.shape
    assert q.shape[:2] == v.shape[:2]
    assert beta.ndim == 2 and g.ndim == 2
    assert beta.shape == g.shape == q.shape[:2]
    assert q.dtype == torch.bfloat16
    assert k.dtype == torch.bfloat16
    assert v.dtype == torch.bfloat16
    assert beta.dtype == torch.float32 and g.dtype == torch.float32
    assert q.device == k.device == v.device == beta.device == g.device
    key_dim = q.shape[2]
    assert key_dim > 0 and (key_dim & (key_dim - 1)) == 0
    assert v.shape[-1] % 128 == 0


def _tensor_args(q, k, v, beta, g, out, state):
    return (
        _lib.ptr(q), _lib.strides(q), _lib.ptr(k), _lib.strides(k), _lib.ptr(v), _lib.strides(v),
        _lib.ptr(beta), _lib.strides(beta), _lib.ptr(g), _lib.strides(g), _lib.ptr(out),
        _lib.strides(out), _lib.ptr(state), _lib.strides(state),
    )


@torch.library.custom_op(
    "wy_lib::gdn_recurrent_prefill_sequential", mutates_args=(), device_types="cuda"
)
def gdn_recurrent_prefill_sequential(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    beta: torch.Tensor,
    g: torch.Tensor,
    cu_seqlens: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Delta-rule recurrence over a prompt.  q, k ``[T, H, DK]``, v ``[T, H, DV]``
    bf16, beta, g ``[T, H]`` fp32.  With ``cu_seqlens`` (``[B+1]`` int32) the
    input is a packed batch, each sequence starting from a zero state, and the
    state is ``[B, H, DK, DV]``; without it one sequence and ``[H, DK, DV]``.
    Returns ``(out [T, H, DV] bf16, state fp32)``."""
    _check_common(q, k, v, beta, g)
    token_num, num_heads, key_dim = q.shape
    value_dim = v.shape[-1]
    assert token_num > 0 and num_heads > 0
    if cu_seqlens is None:
        cu_seqlens = torch.tensor([0, token_num], dtype=torch.int32, device=q.device)
        squeeze_state = True
    else:
        assert cu_seqlens.dtype == torch.int32 and cu_seqlens.ndim == 1
        assert int(cu_seqlens[-1]) == token_num, (
            f"cu_seqlens[-1]={int(cu_seqlens[-1])} does not match the packed token count "
            f"{token_num}"
        )
        cu_seqlens = cu_seqlens.contiguous()
        squeeze_state = False
    batch = cu_seqlens.numel() - 1
    out = torch.empty_like(v)
    state = torch.empty((batch, num_heads, key_dim, value_dim), dtype=torch.float32,
                        device=q.device)
    _lib.call(
        "wy_gdn_recurrent_prefill_sequential", *_tensor_args(q, k, v, beta, g, out, state),
        _lib.ptr(cu_seqlens), batch, num_heads, key_dim, value_dim, _lib.stream(q.device),
    )
    return out, (state[0] if squeeze_state else state)


@gdn_recurrent_prefill_sequential.register_fake
def _gdn_recurrent_prefill_sequential_fake(q, k, v, beta, g, cu_seqlens=None):
    num_heads, key_dim, value_dim = q.shape[1], q.shape[2], v.shape[2]
    shape = ((num_heads, key_dim, value_dim) if cu_seqlens is None
             else (cu_seqlens.numel() - 1, num_heads, key_dim, value_dim))
    return torch.empty_like(v), torch.empty(shape, dtype=torch.float32, device=q.device)


def call_gdn_recurrent_prefill_sequential_triton(q, k, v, beta, g, cu_seqlens=None):
    return gdn_recurrent_prefill_sequential(q, k, v, beta, g, cu_seqlens)


@torch.library.custom_op("wy_lib::gdn_recurrent_decode", mutates_args=("state",),
                         device_types="cuda")
def gdn_recurrent_decode(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    beta: torch.Tensor,
    g: torch.Tensor,
    state: torch.Tensor,
) -> torch.Tensor:
    """One decode token per sequence: q, k ``[B, H, DK]``, v ``[B, H, DV]``
    bf16, beta, g ``[B, H]`` fp32; ``state`` ``[B, H, DK, DV]`` fp32 advanced
    in place.  Returns ``out [B, H, DV]`` bf16."""
    _check_common(q, k, v, beta, g)
    assert state.dtype == torch.float32
    assert q.device == state.device
    batch, num_heads, key_dim = q.shape
    value_dim = v.shape[-1]
    assert state.shape == (batch, num_heads, key_dim, value_dim), (
        f"state must be [B,H,DK,DV]={(batch, num_heads, key_dim, value_dim)}, "
        f"got {tuple(state.shape)}"
    )
    out = torch.empty_like(v)
    _lib.call(
        "wy_gdn_recurrent_decode", *_tensor_args(q, k, v, beta, g, out, state), batch,
        num_heads, key_dim, value_dim, _lib.stream(q.device),
    )
    return out


@gdn_recurrent_decode.register_fake
def _gdn_recurrent_decode_fake(q, k, v, beta, g, state):
    return torch.empty_like(v)


def call_gdn_recurrent_decode_triton(q, k, v, beta, g, state):
    return gdn_recurrent_decode(q, k, v, beta, g, state)
