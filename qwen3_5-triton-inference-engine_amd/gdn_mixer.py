"""The GDN decode mixer between the fused projection and out_proj.

``gdn_decode_ops`` is the reference runner's sequence (engine/runner.py:431-441):
conv4 decode -> q/k norm + gates -> recurrence step -> gated RMSNorm, four
launches.  ``gdn_decode_block`` (op ``wy_lib::gdn_decode_block``) is the same
computation in one launch, bit-identical to the sequence.
"""

from __future__ import annotations

import torch

from . import _lib
from .depthwise_causal_conv4_decode import depthwise_causal_conv4_decode
from .gdn_gated_rmsnorm import gdn_gated_rmsnorm
from .gdn_qk_norm_gates import gdn_qk_norm_gates
from .gdn_recurrent_prefill import gdn_recurrent_decode


def _split_fused(fused: torch.Tensor, heads: int, head_dim: int):
    # column layout of the fused projection (engine/runner.py:424-428)
    key_dim = heads * head_dim
    qkv = fused[:, : 3 * key_dim]
    z = fused[:, 3 * key_dim: 4 * key_dim]
    a = fused[:, 4 * key_dim: 4 * key_dim + heads]
    b = fused[:, 4 * key_dim + heads:]
    return qkv, z, a, b


def gdn_decode_ops(fused, conv_state, conv_weight, a_log, dt_bias, norm_weight,
                   recurrent_state):
    """The runner's four-op GDN decode (engine/runner.py:431-441); returns the
    ``[B, H*D]`` out_proj input and advances both states in place."""
    batch = fused.shape[0]
    heads, head_dim = recurrent_state.shape[1], recurrent_state.shape[2]
    key_dim = heads * head_dim
    qkv, z, a, b = _split_fused(fused, heads, head_dim)
    conv = depthwise_causal_conv4_decode(qkv, conv_state, conv_weight)
    q = conv[:, 0:key_dim].view(batch, heads, head_dim)
    k = conv[:, key_dim: 2 * key_dim].view(batch, heads, head_dim)
    v = conv[:, 2 * key_dim: 3 * key_dim].view(batch, heads, head_dim)
    q_n, k_n, beta, g = gdn_qk_norm_gates(q, k, a, b, a_log, dt_bias)
    core = gdn_recurrent_decode(q_n, k_n, v, beta, g, recurrent_state)
    normed = gdn_gated_rmsnorm(core, z.view(batch, heads, head_dim), norm_weight)
    return normed.view(batch, key_dim)


@torch.library.custom_op("wy_lib::gdn_decode_block",
                         mutates_args=("conv_state", "recurrent_state"), device_types="cuda")
def gdn_decode_block(
    fused: torch.Tensor,
    conv_state: torch.Tensor,
    conv_weight: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    norm_weight: torch.Tensor,
    recurrent_state: torch.Tensor,
) -> torch.Tensor:
    """``gdn_decode_ops`` in one launch.  fused ``[B, 4*H*D + 2*H]`` bf16 (unit
    inner stride); conv_state ``[B, 4, 3*H*D]`` bf16 and conv_weight
    ``[4, 3*H*D]`` bf16 (contiguous); a_log ``[H]`` fp32, dt_bias ``[H]`` bf16,
    norm_weight ``[D]`` fp32; recurrent_state ``[B, H, D, D]`` fp32.  Returns
    ``[B, H*D]`` bf16."""
    assert fused.dtype == conv_state.dtype == conv_weight.dtype == torch.bfloat16
    assert recurrent_state.dtype == torch.float32 and recurrent_state.ndim == 4
    batch, heads, head_dim = recurrent_state.shape[:3]
    assert recurrent_state.shape[3] == head_dim
    key_dim = heads * head_dim
    assert fused.ndim == 2 and fused.shape == (batch, 4 * key_dim + 2 * heads)
    assert fused.stride(1) == 1
    assert conv_state.shape == (batch, 4, 3 * key_dim) and conv_state.is_contiguous()
    assert conv_weight.shape == (4, 3 * key_dim) and conv_weight.is_contiguous()
    assert a_log.dtype == torch.float32 and a_log.shape == (heads,)
    assert dt_bias.dtype == torch.bfloat16 and dt_bias.shape == (heads,)
    assert norm_weight.dtype == torch.float32 and norm_weight.shape == (head_dim,)
    a_log, dt_bias, norm_weight = a_log.contiguous(), dt_bias.contiguous(), norm_weight.contiguous()
    out = torch.empty((batch, key_dim), dtype=fused.dtype, device=fused.device)
    _lib.call(
        "wy_gdn_decode_block", _lib.ptr(fused), fused.stride(0), _lib.ptr(conv_state),
        _lib.strides(conv_state), _lib.ptr(conv_weight), conv_weight.stride(0), _lib.ptr(a_log),
        _lib.ptr(dt_bias), _lib.ptr(norm_weight), _lib.ptr(recurrent_state),
        _lib.strides(recurrent_state), _lib.ptr(out), out.stride(0), batch, heads, head_dim,
        _lib.stream(fused.device),
    )
    return out


@gdn_decode_block.register_fake
def _gdn_decode_block_fake(fused, conv_state, conv_weight, a_log, dt_bias, norm_weight,
                           recurrent_state):
    batch, heads, head_dim = recurrent_state.shape[:3]
    return fused.new_empty((batch, heads * head_dim))
