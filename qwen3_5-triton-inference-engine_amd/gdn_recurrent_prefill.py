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


def gdn_prefill_sequential_into(q, k, v, beta, g, cu_seqlens, state):
    """The packed sequential prefill writing its final states into ``state``
    (``[B, H, DK, DV]`` fp32, e.g. a decoder's recurrent-state cache) instead
    of a new tensor, for callers that validated ``cu_seqlens`` on the host
    (``PackedBatch``): no device-to-host read of ``cu_seqlens[-1]`` and no
    state copy.  Returns ``out [T, H, DV]`` bf16."""
    _check_common(q, k, v, beta, g)
    token_num, num_heads, key_dim = q.shape
    value_dim = v.shape[-1]
    batch = cu_seqlens.numel() - 1
    assert cu_seqlens.dtype == torch.int32 and cu_seqlens.is_contiguous()
    assert state.dtype == torch.float32
    assert state.shape == (batch, num_heads, key_dim, value_dim)
    out = torch.empty_like(v)
    _lib.call(
        "wy_gdn_recurrent_prefill_sequential", *_tensor_args(q, k, v, beta, g, out, state),
        _lib.ptr(cu_seqlens), batch, num_heads, key_dim, value_dim, _lib.stream(q.device),
    )
    return out


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


# ---------------------------------------------------------------- chunk-64 (WY) prefill
CHUNK_SIZE = 64


def _rows16(t):
    """The chunk kernels read 16-byte row chunks: unit inner stride, 16-byte
    aligned rows 8 elements apart; copy otherwise."""
    if t.stride(2) != 1 or t.stride(0) % 8 or t.stride(1) % 8 or t.data_ptr() % 16:
        return t.contiguous()
    return t


@torch.library.custom_op("wy_lib::gdn_chunk_prepare_wy", mutates_args=(), device_types="cuda")
def gdn_chunk_prepare_wy(
    k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor, g: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per 64-token chunk and head: ``(w [N, H, 64, DK], u_base [N, H, 64, DV],
    g_cumsum [N, H, 64])`` fp32 (reference gdn_recurrent_prefill.py:703-826)."""
    assert k.ndim == 3 and v.ndim == 3
    assert k.shape[:2] == v.shape[:2]
    assert beta.ndim == 2 and g.ndim == 2
    assert beta.shape == g.shape == k.shape[:2]
    assert k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16
    assert beta.dtype == torch.float32 and g.dtype == torch.float32
    assert k.device == v.device == beta.device == g.device
    token_num, num_heads, key_dim = k.shape
    value_dim = v.shape[-1]
    assert token_num > 0 and num_heads > 0
    assert key_dim % 16 == 0 and value_dim % 16 == 0
    num_chunks = -(-token_num // CHUNK_SIZE)
    k, v = _rows16(k), _rows16(v)
    w = torch.empty((num_chunks, num_heads, CHUNK_SIZE, key_dim), dtype=torch.float32,
                    device=k.device)
    u_base = torch.empty((num_chunks, num_heads, CHUNK_SIZE, value_dim), dtype=torch.float32,
                         device=k.device)
    g_cumsum = torch.empty((num_chunks, num_heads, CHUNK_SIZE), dtype=torch.float32,
                           device=k.device)
    _lib.call("wy_gdn_chunk_prepare_wy", _lib.ptr(k), _lib.strides(k), _lib.ptr(v),
              _lib.strides(v), _lib.ptr(beta), _lib.strides(beta), _lib.ptr(g), _lib.strides(g),
              _lib.ptr(w), _lib.ptr(u_base), _lib.ptr(g_cumsum), token_num, num_heads, key_dim,
              value_dim, _lib.stream(k.device))
    return w, u_base, g_cumsum


@gdn_chunk_prepare_wy.register_fake
def _gdn_chunk_prepare_wy_fake(k, v, beta, g):
    token_num, num_heads, key_dim = k.shape
    n = -(-token_num // CHUNK_SIZE)
    f = dict(dtype=torch.float32, device=k.device)
    return (torch.empty((n, num_heads, CHUNK_SIZE, key_dim), **f),
            torch.empty((n, num_heads, CHUNK_SIZE, v.shape[-1]), **f),
            torch.empty((n, num_heads, CHUNK_SIZE), **f))


def call_gdn_chunk_prepare_wy_triton(k, v, beta, g):
    return gdn_chunk_prepare_wy(k, v, beta, g)


@torch.library.custom_op("wy_lib::gdn_chunk_state", mutates_args=(), device_types="cuda")
def gdn_chunk_state(
    k: torch.Tensor, w: torch.Tensor, u_base: torch.Tensor, g_cumsum: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """The chunk recurrence: ``(delta [N, H, 64, DV], chunk_state [N, H, DK, DV],
    final_state [H, DK, DV])`` fp32 (reference gdn_recurrent_prefill.py:829-936)."""
    assert k.ndim == 3 and k.dtype == torch.bfloat16
    assert w.ndim == 4 and u_base.ndim == 4 and g_cumsum.ndim == 3
    assert w.dtype == u_base.dtype == g_cumsum.dtype == torch.float32
    assert k.device == w.device == u_base.device == g_cumsum.device
    token_num, num_heads, key_dim = k.shape
    num_chunks, state_heads, chunk_size, state_key_dim = w.shape
    value_dim = u_base.shape[-1]
    assert token_num > 0
    assert state_heads == num_heads and state_key_dim == key_dim
    assert chunk_size == CHUNK_SIZE
    assert u_base.shape == (num_chunks, num_heads, chunk_size, value_dim)
    assert g_cumsum.shape == (num_chunks, num_heads, chunk_size)
    assert num_chunks == -(-token_num // CHUNK_SIZE)
    k = _rows16(k)
    w, u_base, g_cumsum = w.contiguous(), u_base.contiguous(), g_cumsum.contiguous()
    delta = torch.empty_like(u_base)
    chunk_state = torch.empty((num_chunks, num_heads, key_dim, value_dim), dtype=torch.float32,
                              device=k.device)
    final_state = torch.empty((num_heads, key_dim, value_dim), dtype=torch.float32,
                              device=k.device)
    _lib.call("wy_gdn_chunk_state", _lib.ptr(k), _lib.strides(k), _lib.ptr(w), _lib.ptr(u_base),
              _lib.ptr(g_cumsum), _lib.ptr(delta), _lib.ptr(chunk_state), _lib.ptr(final_state),
              token_num, num_heads, key_dim, value_dim, _lib.stream(k.device))
    return delta, chunk_state, final_state


@gdn_chunk_state.register_fake
def _gdn_chunk_state_fake(k, w, u_base, g_cumsum):
    _, num_heads, key_dim = k.shape
    num_chunks, _, _, value_dim = u_base.shape
    f = dict(dtype=torch.float32, device=k.device)
    return (torch.empty_like(u_base), torch.empty((num_chunks, num_heads, key_dim, value_dim), **f),
            torch.empty((num_heads, key_dim, value_dim), **f))


def call_gdn_chunk_state_triton(k, w, u_base, g_cumsum):
    return gdn_chunk_state(k, w, u_base, g_cumsum)


@torch.library.custom_op("wy_lib::gdn_chunk_output", mutates_args=(), device_types="cuda")
def gdn_chunk_output(
    q: torch.Tensor, k: torch.Tensor, delta: torch.Tensor, g_cumsum: torch.Tensor,
    chunk_state: torch.Tensor,
) -> torch.Tensor:
    """``out [T, H, DV]`` bf16 of every chunk (reference gdn_recurrent_prefill.py:939-1023)."""
    assert q.ndim == 3 and k.ndim == 3 and q.shape == k.shape
    assert q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16
    assert delta.ndim == 4 and delta.dtype == torch.float32
    assert g_cumsum.ndim == 3 and g_cumsum.dtype == torch.float32
    assert chunk_state.ndim == 4 and chunk_state.dtype == torch.float32
    assert q.device == k.device == delta.device == g_cumsum.device == chunk_state.device
    token_num, num_heads, key_dim = q.shape
    num_chunks, delta_heads, chunk_size, value_dim = delta.shape
    assert token_num > 0 and delta_heads == num_heads
    assert chunk_size == CHUNK_SIZE
    assert num_chunks == -(-token_num // CHUNK_SIZE)
    assert g_cumsum.shape == (num_chunks, num_heads, chunk_size)
    assert chunk_state.shape == (num_chunks, num_heads, key_dim, value_dim)
    q, k = _rows16(q), _rows16(k)
    delta, g_cumsum, chunk_state = delta.contiguous(), g_cumsum.contiguous(), chunk_state.contiguous()
    out = torch.empty((token_num, num_heads, value_dim), dtype=q.dtype, device=q.device)
    _lib.call("wy_gdn_chunk_output", _lib.ptr(q), _lib.strides(q), _lib.ptr(k), _lib.strides(k),
              _lib.ptr(delta), _lib.ptr(g_cumsum), _lib.ptr(chunk_state), _lib.ptr(out),
              _lib.strides(out), token_num, num_heads, key_dim, value_dim, _lib.stream(q.device))
    return out


@gdn_chunk_output.register_fake
def _gdn_chunk_output_fake(q, k, delta, g_cumsum, chunk_state):
    return torch.empty((q.shape[0], q.shape[1], delta.shape[-1]), dtype=q.dtype, device=q.device)


def call_gdn_chunk_output_triton(q, k, delta, g_cumsum, chunk_state):
    return gdn_chunk_output(q, k, delta, g_cumsum, chunk_state)


def call_gdn_recurrent_prefill_chunked_triton(q, k, v, beta, g):
    """One prompt through the three chunk launches: ``(out [T, H, DV] bf16,
    final_state [H, DK, DV] fp32)`` (reference gdn_recurrent_prefill.py:1026-1048)."""
    w, u_base, g_cumsum = gdn_chunk_prepare_wy(k, v, beta, g)
    delta, chunk_state, final_state = gdn_chunk_state(k, w, u_base, g_cumsum)
    return gdn_chunk_output(q, k, delta, g_cumsum, chunk_state), final_state
