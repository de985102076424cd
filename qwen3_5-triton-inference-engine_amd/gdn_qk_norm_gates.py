"""GDN q/k L2 norm and beta / g gates (MI355X HIP).

Drop-in for ``triton_kernels/gdn_qk_norm_gates.py``: same op name
``wy_lib::gdn_qk_norm_gates``, schema, assertions and outputs (reference
:127-201), plus ``call_gdn_qk_norm_gates_triton`` (:220-229).
"""

from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op("wy_lib::gdn_qk_norm_gates", mutates_args=(), device_types="cuda")
def gdn_qk_norm_gates(
    q: torch.Tensor,
    k: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """q, k ``[T, H, D]`` bf16; a, b ``[T, H]`` bf16; a_log ``[H]`` fp32; dt_bias
    ``[H]`` bf16.  Returns ``(q * rsqrt(|q|^2 + 1e-6) * D^-1/2, k * rsqrt(|k|^2 + 1e-6)``
    (bf16), ``sigmoid(b), -exp(a_log) * softplus(a + dt_bias)`` (fp32 ``[T, H]``)."""
    assert q.ndim == 3 and k.ndim == 3
    assert q.shape == k.shape
    assert a.ndim == 2 and b.ndim == 2 and a.shape == b.shape
    assert a_log.ndim == 1 and dt_bias.ndim == 1
    assert q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16
    assert a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16
    assert a_log.dtype == torch.float32 and dt_bias.dtype == torch.bfloat16
    assert q.device == k.device == a.device == b.device == a_log.device == dt_bias.device
    token_num, num_heads, head_dim = q.shape
    assert token_num > 0
    assert a.shape == (token_num, num_heads)
    assert a_log.shape == (num_heads,) and dt_bias.shape == (num_heads,)
    assert num_heads & (num_heads - 1) == 0
    assert head_dim & (head_dim - 1) == 0
    a_log, dt_bias = a_log.contiguous(), dt_bias.contiguous()
    q_norm = torch.empty((token_num, num_heads, head_dim), dtype=q.dtype, device=q.device)
    k_norm = torch.empty_like(q_norm)
    beta = torch.empty((token_num, num_heads), dtype=torch.float32, device=q.device)
    g = torch.empty_like(beta)
    _lib.call(
        "wy_gdn_qk_norm_gates", _lib.ptr(q), _lib.strides(q), _lib.ptr(k), _lib.strides(k),
        _lib.ptr(a), _lib.strides(a), _lib.ptr(b), _lib.strides(b), _lib.ptr(a_log),
        _lib.ptr(dt_bias), _lib.ptr(q_norm), _lib.ptr(k_norm), _lib.ptr(beta), _lib.ptr(g),
        token_num, num_heads, head_dim, _lib.stream(q.device),
    )
    return q_norm, k_norm, beta, g


@gdn_qk_norm_gates.register_fake
def _gdn_qk_norm_gates_fake(q, k, a, b, a_log, dt_bias):
    token_num, num_heads, head_dim = q.shape
    qn = torch.empty((token_num, num_heads, head_dim), dtype=q.dtype, device=q.device)
    beta = torch.empty((token_num, num_heads), dtype=torch.float32, device=q.device)
    return qn, torch.empty_like(qn), beta, torch.empty_like(beta)


def call_gdn_qk_norm_gates_triton(q, k, a, b, a_log, dt_bias):
    return gdn_qk_norm_gates(q, k, a, b, a_log, dt_bias)
