"""Projection GEMM ``y = x @ weight.T`` on MFMA (MI355X HIP).

Drop-in for ``triton_kernels/gemm_2d.py``: same op name ``wy_lib::gemm_2d``,
schema ``(Tensor x, Tensor weight) -> Tensor``, assertions (bf16 operands,
matching K, ``K % 128 == 0``; reference :197-205) and a fresh contiguous
``[M, N]`` bf16 output, plus ``call_gemm_2d_triton`` (:233-237).  It feeds the
attention block: the fused q/gate/k/v projection before the decode step and
``o_proj`` after the gate pack (engine/runner.py:464, :518; prefill :329-332,
:365).  The kernels need K contiguous in x and weight; other strides are made
contiguous first (the reference kernel reads any strides directly).
"""

from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op("wy_lib::gemm_2d", mutates_args=(), device_types="cuda")
def gemm_2d(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``[M, N] = x [M, K] @ weight [N, K]^T``, fp32 accumulation, bf16 out."""
    assert x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
    assert x.shape[1] == weight.shape[1]
    assert x.shape[1] % 128 == 0
    M, K = x.shape
    N = weight.shape[0]
    if x.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        x = x.contiguous()
    if weight.stride(1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16:
        weight = weight.contiguous()
    out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    # Decode shapes with few column blocks split K across workgroups; the
    # split counters and fp32 partials live in a per-stream workspace.
    ws_bytes = _lib.load().wy_gemm_2d_workspace_bytes(M, N, K)
    ws = _lib.stream_workspace(x.device, "gemm_split", ws_bytes) if ws_bytes > 0 else None
    _lib.call(
        "wy_gemm_2d", _lib.ptr(x), _lib.i64_array(x.stride()), _lib.ptr(weight),
        _lib.i64_array(weight.stride()), _lib.ptr(out), _lib.i64_array(out.stride()),
        M, N, K, _lib.ptr(ws), ws.numel() if ws is not None else 0, _lib.stream(x.device),
    )
    return out


@gemm_2d.register_fake
def _gemm_2d_fake(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    return torch.empty((x.shape[0], weight.shape[0]), dtype=x.dtype, device=x.device)


def call_gemm_2d_triton(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    return gemm_2d(x, weight)
