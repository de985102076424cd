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


def _rows16(t):
    """The fused-prologue kernels read 16-byte chunks of every row: rows must be
    unit-stride, start 16-byte aligned and be 8 elements apart; copy otherwise."""
    if t.stride(1) != 1 or t.stride(0) % 8 or t.data_ptr() % 16:
        return t.contiguous()
    return t


def _split_workspace(x, M, N, K):
    ws_bytes = _lib.load().wy_gemm_2d_workspace_bytes(M, N, K)
    ws = _lib.stream_workspace(x.device, "gemm_split", ws_bytes) if ws_bytes > 0 else None
    return ws, (ws.numel() if ws is not None else 0)


@torch.library.custom_op("wy_lib::rmsnorm_gemm_2d", mutates_args=(), device_types="cuda")
def rmsnorm_gemm_2d(x: torch.Tensor, residual: torch.Tensor | None, norm_weight: torch.Tensor,
                    eps: float, weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``t = x + residual`` (or x), ``y = qwen_rmsnorm(t, norm_weight, eps) @ weight.T``
    in one launch (decode M <= 64); returns ``(y, t)``.  Bit-identical to
    residual_add -> qwen_rmsnorm -> gemm_2d (engine/runner.py:538-562)."""
    assert x.ndim == 2 and x.dtype == weight.dtype == norm_weight.dtype == torch.bfloat16
    assert weight.is_contiguous() and norm_weight.is_contiguous()
    x = _rows16(x)
    M, K = x.shape
    N = weight.shape[0]
    assert weight.shape[1] == K and norm_weight.shape == (K,) and K % 256 == 0 and M <= 64
    if residual is not None:
        assert residual.shape == x.shape and residual.dtype == x.dtype
        residual = _rows16(residual)
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    t = torch.empty((M, K), dtype=x.dtype, device=x.device) if residual is not None else None
    ws, nbytes = _split_workspace(x, M, N, K)
    _lib.call("wy_gemm_2d_rmsnorm", _lib.ptr(x), x.stride(0), _lib.ptr(residual),
              residual.stride(0) if residual is not None else 0, _lib.ptr(norm_weight),
              float(eps), _lib.ptr(t), K, _lib.ptr(weight), weight.stride(0), _lib.ptr(y),
              y.stride(0), M, N, K, _lib.ptr(ws), nbytes, _lib.stream(x.device))
    return y, (t if t is not None else x.clone())


@rmsnorm_gemm_2d.register_fake
def _rmsnorm_gemm_2d_fake(x, residual, norm_weight, eps, weight):
    return x.new_empty((x.shape[0], weight.shape[0])), torch.empty_like(x)


@torch.library.custom_op("wy_lib::swiglu_gemm_2d", mutates_args=(), device_types="cuda")
def swiglu_gemm_2d(gate_up: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``swiglu(gate_up[:, :I], gate_up[:, I:]) @ weight.T`` (I = weight.shape[1])
    in one launch (M <= 64); bit-identical to swiglu -> gemm_2d
    (engine/runner.py:562-565)."""
    assert gate_up.ndim == 2 and gate_up.dtype == weight.dtype == torch.bfloat16
    assert weight.is_contiguous()
    gate_up = _rows16(gate_up)
    M = gate_up.shape[0]
    N, K = weight.shape
    assert gate_up.shape[1] == 2 * K and K % 128 == 0 and M <= 64
    y = torch.empty((M, N), dtype=gate_up.dtype, device=gate_up.device)
    ws, nbytes = _split_workspace(gate_up, M, N, K)
    _lib.call("wy_gemm_2d_swiglu", _lib.ptr(gate_up), gate_up.stride(0), K, _lib.ptr(weight),
              weight.stride(0), _lib.ptr(y), y.stride(0), M, N, K, _lib.ptr(ws), nbytes,
              _lib.stream(gate_up.device))
    return y


@swiglu_gemm_2d.register_fake
def _swiglu_gemm_2d_fake(gate_up, weight):
    return gate_up.new_empty((gate_up.shape[0], weight.shape[0]))


@torch.library.custom_op("wy_lib::gate_up_swiglu", mutates_args=(), device_types="cuda")
def gate_up_swiglu(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``swiglu(g, u)`` of ``[g | u] = x @ weight.T`` (weight ``[2I, K]``: gate
    rows then up rows), ``[M, I]`` bf16, in one launch with SwiGLU in the GEMM
    epilogue (decode rows M <= 64 on the skinny kernel, more rows on the tile
    kernel when I % 128 == 0; other shapes run gemm_2d then swiglu).
    Bit-identical to gemm_2d -> swiglu except for M <= 64 with 2I < 4096
    (engine/runner.py:560-565)."""
    from .swiglu import swiglu

    assert x.ndim == 2 and x.dtype == weight.dtype == torch.bfloat16
    assert weight.is_contiguous() and weight.shape[0] % 2 == 0
    M, K = x.shape
    N = weight.shape[0] // 2
    assert weight.shape[1] == K and K % 128 == 0
    if M > 64 and N % 128:
        gu = gemm_2d(x, weight)
        return swiglu(gu[:, :N], gu[:, N:])
    x = _rows16(x)
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    ws_bytes = _lib.load().wy_gemm_2d_gate_up_swiglu_workspace_bytes(M, N, K)
    ws = _lib.stream_workspace(x.device, "gemm_split", ws_bytes) if ws_bytes > 0 else None
    _lib.call("wy_gemm_2d_gate_up_swiglu", _lib.ptr(x), x.stride(0), _lib.ptr(weight),
              weight.stride(0), _lib.ptr(y), y.stride(0), M, N, K, _lib.ptr(ws),
              ws.numel() if ws is not None else 0, _lib.stream(x.device))
    return y


@gate_up_swiglu.register_fake
def _gate_up_swiglu_fake(x, weight):
    return x.new_empty((x.shape[0], weight.shape[0] // 2))
