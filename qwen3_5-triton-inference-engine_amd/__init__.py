"""MI355X (gfx950) full-attention hot path of the Qwen3.5 inference engine.

Hand-written HIP kernels behind the reference engine's ``wy_lib::`` torch ops.
Module names mirror the reference's ``triton_kernels/`` files so a caller
switches by import path only; ``install_as_triton_kernels()`` makes the
reference's own import lines resolve to these modules.
"""

from __future__ import annotations

import sys

from . import _lib
from .attention import (
    PackedBatch,
    build_packed_batch,
    decode_attention_block,
    decode_attention_step,
    prefill_attention_block,
    prefill_attention_packed,
)
from .attention_gate_pack import attention_gate_pack
from .cache import AttnCaches, allocate_attn_caches
from .decoder import DecodeModel, DecoderConfig, GraphedDecoder, random_weights
from .embedding_gather import call_embedding_gather_triton, embedding_gather
from .gemm_2d import (call_gemm_2d_triton, gate_up_swiglu, gemm_2d, rmsnorm_gemm_2d,
                      swiglu_gemm_2d)
from .gqa_attention_decode_paged import (
    MAX_SPLITS,
    MIN_PAGES_PER_SPLIT,
    PAGE_SIZE,
    allocate_paged_kv_cache,
    allocate_split_scratch,
    call_paged_gqa_attention_decode_triton,
    SplitScratch,
    paged_gqa_attention_decode_block,
    paged_gqa_attention_decode_combine,
    paged_gqa_attention_decode_fused,
    paged_gqa_attention_decode_split,
    paged_kv_append,
    paged_kv_fill,
    paged_kv_fill_varlen,
    page_stream_read,
    physical_rows,
)
from .depthwise_causal_conv4_decode import (
    call_depthwise_causal_conv4_decode_triton,
    conv_state_from_packed_prefill,
    conv_state_from_prefill,
    depthwise_causal_conv4_decode,
)
from .depthwise_causal_conv4_prefill import (
    build_seq_start,
    call_depthwise_causal_conv4_prefill_triton,
    depthwise_causal_conv4_prefill,
)
from .gdn_gated_rmsnorm import call_gdn_gated_rmsnorm_triton, gdn_gated_rmsnorm
from .gdn_mixer import gdn_decode_block, gdn_decode_ops
from .gdn_qk_norm_gates import call_gdn_qk_norm_gates_triton, gdn_qk_norm_gates
from .gdn_recurrent_prefill import (
    call_gdn_chunk_output_triton,
    call_gdn_chunk_prepare_wy_triton,
    call_gdn_chunk_state_triton,
    call_gdn_recurrent_decode_triton,
    call_gdn_recurrent_prefill_chunked_triton,
    call_gdn_recurrent_prefill_sequential_triton,
    gdn_chunk_output,
    gdn_chunk_prepare_wy,
    gdn_chunk_state,
    gdn_recurrent_decode,
    gdn_recurrent_prefill_sequential,
)
from .gqa_attention_varlen_causal import build_cu_seqlens, gqa_attention_varlen_causal
from .paging import PagePool, SequencePages, allocate_block_table
from .partial_rope import partial_rope, rope_inv_freq
from .qwen_rmsnorm import add_rmsnorm, call_qwen_rmsnorm_triton, qwen_rmsnorm
from .residual_add import call_residual_add_triton, residual_add
from .swiglu import call_swiglu_triton, swiglu
from .vocab_argmax import call_lm_head_argmax_triton, lm_head_argmax


def install_as_triton_kernels() -> None:
    """Alias the reference module paths (``triton_kernels.<op>`` and
    ``engine.paging``) to this package's modules in ``sys.modules``."""
    import importlib
    for name, sub in (
        ("triton_kernels.gqa_attention_decode_paged", "gqa_attention_decode_paged"),
        ("triton_kernels.gqa_attention_varlen_causal", "gqa_attention_varlen_causal"),
        ("triton_kernels.partial_rope", "partial_rope"),
        ("triton_kernels.attention_gate_pack", "attention_gate_pack"),
        ("triton_kernels.qwen_rmsnorm", "qwen_rmsnorm"),
        ("triton_kernels.gemm_2d", "gemm_2d"),
        ("triton_kernels.gdn_recurrent_prefill", "gdn_recurrent_prefill"),
        ("triton_kernels.gdn_qk_norm_gates", "gdn_qk_norm_gates"),
        ("triton_kernels.gdn_gated_rmsnorm", "gdn_gated_rmsnorm"),
        ("triton_kernels.depthwise_causal_conv4_decode", "depthwise_causal_conv4_decode"),
        ("triton_kernels.depthwise_causal_conv4_prefill", "depthwise_causal_conv4_prefill"),
        ("triton_kernels.embedding_gather", "embedding_gather"),
        ("triton_kernels.residual_add", "residual_add"),
        ("triton_kernels.swiglu", "swiglu"),
        ("triton_kernels.vocab_argmax", "vocab_argmax"),
        ("engine.paging", "paging"),
    ):
        # the submodule itself: several share their name with the op they define
        sys.modules[name] = importlib.import_module(f"{__name__}.{sub}")


def library_loaded() -> bool:
    return _lib._lib is not None
