"""ctypes binding of ``lib/libwy_attn.so`` (declared in include/wy_attn.h).

This module is the only place that touches the C ABI.  There is no fallback:
if the library is missing or a call returns an error, a RuntimeError is
raised.  Strides cross the boundary as int64 arrays in elements, streams as
the raw ``hipStream_t`` of torch's current stream.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libwy_attn.so"

_c_i64p = ctypes.POINTER(ctypes.c_int64)
_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float

# name -> argtypes (all return int status)
_SIGNATURES = {
    "wy_paged_kv_append": [_vp, _vp, _c_i64p, _c_i64p, _vp, _vp, _c_i64p, _c_i64p, _vp,
                           _i64, _vp, _i, _i, _i, _vp],
    "wy_paged_kv_fill_varlen": [_vp, _vp, _c_i64p, _c_i64p, _vp, _vp, _c_i64p, _c_i64p,
                                _vp, _i64, _vp, _i, _i, _i, _i, _vp],
    "wy_paged_decode_split": [_vp, _c_i64p, _vp, _vp, _c_i64p, _c_i64p, _vp, _i64, _vp,
                              _vp, _vp, _vp, _c_i64p, _c_i64p, _i, _i, _i, _i, _i, _i,
                              _vp],
    "wy_paged_decode_combine": [_vp, _vp, _vp, _c_i64p, _c_i64p, _vp, _vp, _c_i64p, _i,
                                _i, _i, _i, _vp],
    "wy_paged_decode_step": [_vp, _c_i64p, _vp, _vp, _c_i64p, _c_i64p, _vp, _vp, _c_i64p,
                             _c_i64p, _vp, _i64, _vp, _vp, _vp, _vp, _c_i64p, _c_i64p, _vp,
                             _vp, _c_i64p, _vp, _c_i64p, _i, _i, _i, _i, _i, _i, _vp],
    "wy_paged_decode_step_noalloc": [_vp, _c_i64p, _vp, _vp, _c_i64p, _c_i64p, _vp, _vp,
                                     _c_i64p, _c_i64p, _vp, _i64, _vp, _vp, _c_i64p, _vp,
                                     _c_i64p, _i, _i, _i, _i, _i, _i, _vp],
    "wy_page_stream_read": [_vp, _vp, _c_i64p, _c_i64p, _vp, _i64, _vp, _i, _i, _i, _vp, _vp],
    "wy_gdn_chunk_prepare_wy": [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp,
                                _vp, _vp, _i, _i, _i, _i, _vp],
    "wy_gdn_chunk_state": [_vp, _c_i64p, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "wy_gdn_chunk_output": [_vp, _c_i64p, _vp, _c_i64p, _vp, _vp, _vp, _vp, _c_i64p, _i, _i,
                            _i, _i, _vp],
    "wy_varlen_causal_prefill": [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p,
                                 _vp, _i, _i, _i, _i, _i, _i64, _vp, _i64, _vp],
    "wy_partial_rope": [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _i, _vp, _i, _i, _i, _i,
                        _i, _vp],
    "wy_attention_gate_pack": [_vp, _c_i64p, _vp, _c_i64p, _vp, _i, _i, _i, _vp],
    "wy_qwen_rmsnorm": [_vp, _c_i64p, _vp, _vp, _c_i64p, _i, _i, _i, _f, _vp],
    "wy_prefill_attention_block": [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p,
                                   _vp, _i64, _i, _vp, _i, _vp, _vp, _c_i64p, _c_i64p, _vp,
                                   _i64, _vp, _i, _i, _i, _i, _i, _i64, _vp, _vp, _vp, _vp,
                                   _i64, _vp],
    "wy_prefill_kv_rope_fill": [_vp, _vp, _c_i64p, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp,
                                _c_i64p, _vp, _vp, _i64, _vp, _vp, _i64, _i, _vp, _i, _i, _i,
                                _i, _i, _vp],
    "wy_gemm_2d": [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _i, _i, _i, _vp, _i64, _vp],
    "wy_paged_decode_block": [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp,
                              _vp, _f, _vp, _i, _vp, _vp, _c_i64p, _c_i64p, _vp, _i64, _vp,
                              _vp, _vp, _vp, _c_i64p, _c_i64p, _vp, _vp, _c_i64p, _i, _i,
                              _i, _i, _i, _i, _vp],
    "wy_gdn_recurrent_decode": [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp,
                                _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _i, _i, _i, _i, _vp],
    "wy_gdn_recurrent_prefill_sequential": [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp,
                                            _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p,
                                            _vp, _i, _i, _i, _i, _vp],
    "wy_depthwise_causal_conv4_decode": [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp,
                                         _c_i64p, _i, _i, _vp],
    "wy_gdn_qk_norm_gates": [_vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _c_i64p, _vp, _vp,
                             _vp, _vp, _vp, _vp, _i, _i, _i, _vp],
    "wy_gdn_gated_rmsnorm": [_vp, _c_i64p, _vp, _c_i64p, _vp, _vp, _i, _i, _i, _vp],
    "wy_gdn_decode_block": [_vp, _i64, _vp, _c_i64p, _vp, _i64, _vp, _vp, _vp, _vp, _c_i64p,
                            _vp, _i64, _i, _i, _i, _vp],
    "wy_depthwise_causal_conv4_prefill": [_vp, _c_i64p, _vp, _i64, _i64, _vp, _c_i64p, _vp,
                                          _i, _i, _vp],
    "wy_conv_state_from_packed_prefill": [_vp, _c_i64p, _vp, _c_i64p, _vp, _i, _i, _vp],
    "wy_embedding_gather": [_vp, _i, _vp, _i64, _i64, _vp, _i64, _i, _i, _vp],
    "wy_residual_add": [_vp, _vp, _vp, _i64, _vp],
    "wy_add_rmsnorm": [_vp, _vp, _vp, _vp, _vp, _i, _i, _f, _vp],
    "wy_swiglu": [_vp, _c_i64p, _vp, _c_i64p, _vp, _i, _i, _vp],
    "wy_lm_head_argmax": [_vp, _i64, _vp, _i64, _vp, _i, _i, _i, _vp, _i64, _vp],
    "wy_gemm_2d_rmsnorm": [_vp, _i64, _vp, _i64, _vp, _f, _vp, _i64, _vp, _i64, _vp, _i64, _i,
                           _i, _i, _vp, _i64, _vp],
    "wy_gemm_2d_swiglu": [_vp, _i64, _i64, _vp, _i64, _vp, _i64, _i, _i, _i, _vp, _i64, _vp],
    "wy_gemm_2d_gate_up_swiglu": [_vp, _i64, _vp, _i64, _vp, _i64, _i, _i, _i, _vp, _i64, _vp],
}

# entry points returning a size (int64) rather than a status
_SIZE_QUERIES = ("wy_varlen_causal_prefill_workspace_bytes", "wy_gemm_2d_workspace_bytes",
                 "wy_gemm_2d_gate_up_swiglu_workspace_bytes",
                 "wy_lm_head_argmax_workspace_bytes", "wy_paged_decode_step_noalloc_max_rows",
                 "wy_page_stream_read_waves")

# test hooks returning nothing
_HOOKS = ("wy_prefill_set_ticket_order", "wy_prefill_set_short_path")

EXPORTED = ("wy_status_string", "wy_build_info", *_SIGNATURES, *_SIZE_QUERIES, *_HOOKS)

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build the HIP extension first "
            "(python qwen3_5-triton-inference-engine_amd/build.py)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    lib.wy_status_string.argtypes = [ctypes.c_int]
    lib.wy_status_string.restype = ctypes.c_char_p
    lib.wy_build_info.argtypes = []
    lib.wy_build_info.restype = ctypes.c_char_p
    for fn in (lib.wy_varlen_causal_prefill_workspace_bytes, lib.wy_gemm_2d_workspace_bytes,
               lib.wy_gemm_2d_gate_up_swiglu_workspace_bytes,
               lib.wy_lm_head_argmax_workspace_bytes):
        fn.argtypes = [_i, _i, _i]
        fn.restype = ctypes.c_int64
    for fn in (lib.wy_paged_decode_step_noalloc_max_rows, lib.wy_page_stream_read_waves):
        fn.argtypes = []
        fn.restype = ctypes.c_int64
    lib.wy_prefill_set_ticket_order.argtypes = [_i]
    lib.wy_prefill_set_ticket_order.restype = None
    lib.wy_prefill_set_short_path.argtypes = [_i]
    lib.wy_prefill_set_short_path.restype = None
    _lib = lib
    return lib


def strides(t):
    if t is None:
        return None
    s = t.stride()
    return (ctypes.c_int64 * len(s))(*s)


def i64_array(values):
    return (ctypes.c_int64 * len(values))(*values)


def ptr(t):
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.wy_status_string(rc).decode()
        raise RuntimeError(f"{name} failed with code {rc}: {msg}")


# Device workspaces that must start zeroed and that the kernels leave zeroed
# (ticket / split counters), one per (device, stream, use).  Launches on one
# stream run in order, so they can share one.  A larger request allocates a
# new buffer; the old ones stay referenced, since a captured graph may still
# hold their addresses.
_WORKSPACES: dict = {}


def stream_workspace(device, tag: str, nbytes: int) -> torch.Tensor:
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx, stream(dev), tag)
    bufs = _WORKSPACES.setdefault(key, [])
    if not bufs or bufs[-1].numel() < nbytes:
        size = max(nbytes, 2 * bufs[-1].numel()) if bufs else nbytes
        bufs.append(torch.zeros(size, dtype=torch.uint8, device=dev))
    return bufs[-1]
