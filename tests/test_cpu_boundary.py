"""CPU-side checks: the C-ABI library loads and exports every entry point of
include/wy_attn.h, argument rejection happens before any device work, host
paging logic, fixture integrity.  No kernel runs here."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from tests.golden import cases as C

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "wy_attn.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int64_t|int|void|size_t|const char \*)\s*(wy_\w+)\(", text, re.M)))


def test_header_declares_expected_entry_points():
    names = _declared()
    assert "wy_paged_decode_split" in names and "wy_varlen_causal_prefill" in names
    assert len(names) >= 9


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg._lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_declared()) == set(pkg._lib.EXPORTED)
    assert lib.wy_build_info().decode().endswith("gfx950")


def test_noalloc_step_rejects_over_capacity_before_any_launch(pkg):
    """The scratch-free decode step refuses batch * num_q_heads above its static
    capacity with WY_E_CAPACITY before touching the GPU (safe without one)."""
    lib = pkg._lib.load()
    cap = lib.wy_paged_decode_step_noalloc_max_rows()
    assert cap == 512
    d = ctypes.c_void_p(16)
    s3, s4 = pkg._lib.i64_array([2048, 256, 1]), pkg._lib.i64_array([8192, 4096, 256, 1])
    rc = lib.wy_paged_decode_step_noalloc(d, s3, d, d, s3, s3, d, d, s4, s4, d, 1, d, None,
                                          None, d, s3, cap // 8 + 1, 8, 2, 256, 1, 16, None)
    assert rc == -5 and b"capacity" in lib.wy_status_string(rc)


def test_fused_decoder_entry_points_reject_before_launch(pkg):
    """wy_add_rmsnorm and wy_gemm_2d_gate_up_swiglu refuse NULL, unsupported
    widths and misaligned rows before any launch (safe without a GPU)."""
    lib = pkg._lib.load()
    d, odd = ctypes.c_void_p(4096), ctypes.c_void_p(4098)
    assert lib.wy_add_rmsnorm(None, d, d, d, d, 4, 1024, 1e-6, None) == -1
    assert lib.wy_add_rmsnorm(d, d, d, d, d, 4, 1000, 1e-6, None) == -4   # not % 256
    assert lib.wy_add_rmsnorm(d, d, d, d, d, 4, 2048, 1e-6, None) == -4   # > 1024
    assert lib.wy_add_rmsnorm(d, odd, d, d, d, 4, 1024, 1e-6, None) == -3
    assert lib.wy_add_rmsnorm(d, d, d, d, d, -1, 1024, 1e-6, None) == -2
    assert lib.wy_add_rmsnorm(d, d, d, d, d, 0, 1024, 1e-6, None) == 0    # nothing to do
    g = lib.wy_gemm_2d_gate_up_swiglu
    assert g(None, 1024, d, 1024, d, 3584, 4, 3584, 1024, None, 0, None) == -1
    assert g(d, 1024, d, 1024, d, 3584, 4, 3584, 1000, None, 0, None) == -2   # K % 128
    assert g(d, 1024, d, 1024, d, 1000, 100, 1000, 1024, None, 0, None) == -4  # M > 64, N % 128
    assert g(odd, 1024, d, 1024, d, 3584, 4, 3584, 1024, None, 0, None) == -3
    assert g(d, 1024, d, 1024, d, 3584, 4, 3584, 1024, None, 64, None) == -3  # bytes, no buffer
    assert g(d, 1024, d, 1024, d, 3584, 0, 3584, 1024, None, 0, None) == 0
    assert lib.wy_gemm_2d_gate_up_swiglu_workspace_bytes(32, 3584, 1024) == 0  # no split
    assert lib.wy_gemm_2d_gate_up_swiglu_workspace_bytes(32, 1024, 2048) > 0   # split K
    assert lib.wy_gemm_2d_gate_up_swiglu_workspace_bytes(100, 1024, 2048) == 0  # tile kernel


def test_null_and_unsupported_arguments_are_rejected(pkg):
    lib = pkg._lib.load()
    s4 = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    s3 = (ctypes.c_int64 * 3)(1, 1, 1)
    rc = lib.wy_paged_kv_append(None, None, s4, s4, None, None, s3, s3, None, 0, None,
                                1, 2, 256, None)
    assert rc == -1
    assert "NULL" in lib.wy_status_string(rc).decode()
    dummy = ctypes.c_void_p(16)
    # head_dim 128 has no decode kernel: rejected before launch
    rc = lib.wy_paged_decode_split(dummy, s3, dummy, dummy, s4, s4, dummy, 1, dummy, dummy,
                                   dummy, dummy, s3, s4, 1, 8, 2, 128, 4, 4, None)
    assert rc == -4
    rc = lib.wy_varlen_causal_prefill(dummy, s3, dummy, s3, dummy, s3, dummy, s3, dummy,
                                      1, 8, 2, 64, 16, 16, None, 0, None)
    assert rc == -4
    # prefill: a workspace size without a workspace, or a misaligned one
    s3p = (ctypes.c_int64 * 3)(2048, 256, 1)
    s3k = (ctypes.c_int64 * 3)(512, 256, 1)
    for ws, nbytes in ((None, 64), (ctypes.c_void_p(18), 64), (dummy, -1)):
        rc = lib.wy_varlen_causal_prefill(dummy, s3p, dummy, s3k, dummy, s3k, dummy, s3p, dummy,
                                          1, 8, 2, 256, 16, 16, ws, nbytes, None)
        assert rc == -3
    # prefill block: rotary widths other than 64 are unsupported; NULL gate
    pos = ctypes.c_void_p(64)
    args = [dummy, s3p, dummy, s3k, dummy, s3k, dummy, s3p, pos, 1, 0, dummy]
    tail = [dummy, dummy, s4, s4, dummy, 4, dummy, 1, 8, 2, 256, 16, 16, dummy, dummy, dummy,
            None, 0, None]
    assert lib.wy_prefill_attention_block(*args, 32, *tail) == -4
    args[6] = None
    assert lib.wy_prefill_attention_block(*args, 64, *tail) == -1
    # no work list for an empty launch
    assert lib.wy_varlen_causal_prefill_workspace_bytes(0, 2, 4096) == 0
    assert lib.wy_varlen_causal_prefill_workspace_bytes(4, 2, 0) == 0
    # qwen_rmsnorm: NULL weight; d_model 384 is not a multiple of 256
    assert lib.wy_qwen_rmsnorm(dummy, s3, None, dummy, s3, 1, 1, 256, 1e-6, None) == -1
    assert lib.wy_qwen_rmsnorm(dummy, s3, dummy, dummy, s3, 1, 1, 384, 1e-6, None) == -4
    # decode block: rotary_dim above 128 or not a multiple of 16 is unsupported
    for rd, want in ((256, -4), (72, -4)):
        rc = lib.wy_paged_decode_block(dummy, s3, dummy, s3, dummy, s3, dummy, s3, dummy, dummy,
                                       1e-6, dummy, rd, dummy, dummy, s4, s4, dummy, 1, dummy,
                                       dummy, dummy, dummy, s3, s4, dummy, dummy, s3, 1, 8, 2,
                                       256, 4, 4, None)
        assert rc == want, (rd, rc)
    rc = lib.wy_paged_decode_block(dummy, s3, None, s3, dummy, s3, dummy, s3, dummy, dummy,
                                   1e-6, dummy, 64, dummy, dummy, s4, s4, dummy, 1, dummy,
                                   dummy, dummy, dummy, s3, s4, dummy, dummy, s3, 1, 8, 2,
                                   256, 4, 4, None)
    assert rc == -1  # the gate is required
    rc = lib.wy_partial_rope(dummy, s4, dummy, s4, dummy, (ctypes.c_int64 * 2)(1, 1), 0,
                             dummy, 1, 1, 1, 256, 65, None)
    assert rc == -2  # odd rotary_dim
    # gemm_2d: K not a multiple of 128; a transposed (non K-contiguous) weight
    s2 = (ctypes.c_int64 * 2)(256, 1)
    assert lib.wy_gemm_2d(dummy, s2, dummy, s2, dummy, s2, 4, 8, 200, None, 0, None) == -2
    assert lib.wy_gemm_2d(dummy, s2, None, s2, dummy, s2, 4, 8, 256, None, 0, None) == -1
    assert lib.wy_gemm_2d(dummy, s2, dummy, (ctypes.c_int64 * 2)(1, 256), dummy, s2, 4, 8, 256,
                          None, 0, None) == -3
    # a workspace size without a workspace; a misaligned workspace
    assert lib.wy_gemm_2d(dummy, s2, dummy, s2, dummy, s2, 4, 8, 256, None, 64, None) == -3
    assert lib.wy_gemm_2d(dummy, s2, dummy, s2, dummy, s2, 4, 8, 256, ctypes.c_void_p(18), 64,
                          None) == -3
    assert lib.wy_gemm_2d(dummy, s2, dummy, s2, dummy, s2, 0, 8, 256, None, 0, None) == 0  # empty


def test_gdn_entry_points_reject_before_launch(pkg):
    lib = pkg._lib.load()
    d = ctypes.c_void_p(256)
    s3 = (ctypes.c_int64 * 3)(2048, 128, 1)
    s2 = (ctypes.c_int64 * 2)(16, 1)
    s4 = (ctypes.c_int64 * 4)(16 * 128 * 128, 128 * 128, 128, 1)
    base = [d, s3, d, s3, d, s3, d, s2, d, s2, d, s3, d, s4]
    # key_dim 64 has no kernel
    assert lib.wy_gdn_recurrent_decode(*base, 2, 16, 64, 128, None) == -4
    assert lib.wy_gdn_recurrent_prefill_sequential(*base, d, 2, 16, 64, 128, None) == -4
    # value_dim not a multiple of 128
    assert lib.wy_gdn_recurrent_decode(*base, 2, 16, 128, 96, None) == -4
    # NULL cu_seqlens / NULL state
    assert lib.wy_gdn_recurrent_prefill_sequential(*base, None, 2, 16, 128, 128, None) == -1
    nul = list(base)
    nul[12] = None
    assert lib.wy_gdn_recurrent_decode(*nul, 2, 16, 128, 128, None) == -1
    # state with a non-unit inner stride
    bad = list(base)
    bad[13] = (ctypes.c_int64 * 4)(16 * 128 * 128, 128 * 128, 128, 2)
    assert lib.wy_gdn_recurrent_decode(*bad, 2, 16, 128, 128, None) == -3
    assert lib.wy_gdn_qk_norm_gates(d, s3, d, s3, d, s2, d, s2, d, d, d, d, d, d, 4, 16, 64,
                                    None) == -4
    assert lib.wy_gdn_gated_rmsnorm(d, s3, d, s3, d, d, 4, 16, 256, None) == -4
    cs = (ctypes.c_int64 * 3)(4 * 6144, 6144, 1)
    assert lib.wy_gdn_decode_block(d, 8224, d, cs, d, 6144, d, d, d, d, s4, d, 2048, 2, 16, 64,
                                   None) == -4
    assert lib.wy_gdn_decode_block(None, 8224, d, cs, d, 6144, d, d, d, d, s4, d, 2048, 2, 16,
                                   128, None) == -1
    assert lib.wy_depthwise_causal_conv4_decode(d, s2, d, (ctypes.c_int64 * 3)(4, 1, 2), d, s2,
                                                d, s2, 2, 6144, None) == -3


def test_fused_gemm_and_lm_head_reject_before_launch(pkg):
    lib = pkg._lib.load()
    d = ctypes.c_void_p(256)
    # M > 64 has no fused-prologue kernel; K % 256 for the RMSNorm prologue
    assert lib.wy_gemm_2d_rmsnorm(d, 1024, None, 0, d, 1e-6, None, 0, d, 1024, d, 1024, 65,
                                  1024, 1024, None, 0, None) == -4
    assert lib.wy_gemm_2d_rmsnorm(d, 1024, None, 0, d, 1e-6, None, 0, d, 1024, d, 1024, 4,
                                  1024, 1000, None, 0, None) == -2
    assert lib.wy_gemm_2d_swiglu(d, 7168, 3584, d, 3584, d, 1024, 65, 1024, 3584, None, 0,
                                 None) == -4
    # up half overlapping the gate half
    assert lib.wy_gemm_2d_swiglu(d, 7168, 1024, d, 3584, d, 1024, 4, 1024, 3584, None, 0,
                                 None) == -3
    # more than 64 rows, no workspace, unsupported hidden size
    assert lib.wy_lm_head_argmax(d, 1024, d, 1024, d, 65, 1024, 5000, d, 1 << 20, None) == -2
    assert lib.wy_lm_head_argmax(d, 1024, d, 1024, d, 4, 1024, 5000, None, 0, None) == -1
    assert lib.wy_lm_head_argmax(d, 1024, d, 1024, d, 4, 1000, 5000, d, 1 << 20, None) == -4
    assert lib.wy_lm_head_argmax_workspace_bytes(32, 1024, 248320) > 0


def test_gemm_split_workspace_sizes(pkg):
    """Decode o_proj [1024, 2048] at B=32 splits K 4 ways: 16 KiB of counters
    plus 4 * 32 * 1024 fp32 partials; prefill shapes and wide N do not split."""
    lib = pkg._lib.load()
    assert lib.wy_gemm_2d_workspace_bytes(32, 1024, 2048) == 16384 + 4 * 32 * 1024 * 4
    assert lib.wy_gemm_2d_workspace_bytes(4096, 1024, 2048) == 0
    assert lib.wy_gemm_2d_workspace_bytes(32, 65536, 1024) == 0
    assert lib.wy_gemm_2d_workspace_bytes(32, 1024, 200) == 0


def test_ops_refuse_cpu_tensors(pkg):
    x = torch.zeros(1, 2, 3, 256, dtype=torch.bfloat16)
    with pytest.raises(Exception):
        pkg.attention_gate_pack(x, x)
    with pytest.raises(Exception):
        pkg.partial_rope(x, torch.zeros(1, 3, dtype=torch.int64), torch.zeros(32), 64)


def test_op_schemas_match_reference():
    import __graft_entry__

    __graft_entry__.load_package()
    schemas = {
        "paged_kv_append": "(Tensor(a0!) k_cache, Tensor(a1!) v_cache, Tensor k_new, "
                           "Tensor v_new, Tensor block_table, Tensor pos) -> ()",
        "gqa_attention_varlen_causal": "(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens, "
                                       "SymInt max_seqlen) -> Tensor",
        "attention_gate_pack": "(Tensor x, Tensor gate) -> Tensor",
        "qwen_rmsnorm": "(Tensor x, Tensor weight, float eps=9.9999999999999995e-07) -> Tensor",
        "gemm_2d": "(Tensor x, Tensor weight) -> Tensor",
        "gdn_recurrent_decode": "(Tensor q, Tensor k, Tensor v, Tensor beta, Tensor g, "
                                "Tensor(a5!) state) -> Tensor",
        "gdn_recurrent_prefill_sequential": "(Tensor q, Tensor k, Tensor v, Tensor beta, "
                                            "Tensor g, Tensor? cu_seqlens=None) "
                                            "-> (Tensor, Tensor)",
        "gdn_qk_norm_gates": "(Tensor q, Tensor k, Tensor a, Tensor b, Tensor a_log, "
                             "Tensor dt_bias) -> (Tensor, Tensor, Tensor, Tensor)",
        "gdn_gated_rmsnorm": "(Tensor x, Tensor z, Tensor weight) -> Tensor",
        "depthwise_causal_conv4_decode": "(Tensor x, Tensor(a1!) state, Tensor weight) -> Tensor",
        "depthwise_causal_conv4_prefill": "(Tensor x, Tensor weight, Tensor? seq_start=None) "
                                          "-> Tensor",
        "conv_state_from_packed_prefill": "(Tensor(a0!) state, Tensor x, Tensor cu_seqlens) -> ()",
    }
    for name, sig in schemas.items():
        op = getattr(torch.ops.wy_lib, name).default
        s = str(op._schema)
        assert s.startswith(f"wy_lib::{name}"), s
        args = s[len(f"wy_lib::{name}"):]
        assert args.replace("SymInt", "int") == sig.replace("SymInt", "int"), s
    for name in ("paged_kv_fill_varlen", "paged_gqa_attention_decode_split",
                 "paged_gqa_attention_decode_combine", "partial_rope",
                 "prefill_attention_block", "gdn_decode_block", "rmsnorm_gemm_2d",
                 "swiglu_gemm_2d", "embedding_gather", "residual_add", "swiglu",
                 "lm_head_argmax", "add_rmsnorm", "gate_up_swiglu"):
        assert hasattr(torch.ops.wy_lib, name)


def test_fake_impls_give_reference_shapes(pkg):
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty(1, 8, 5, 256, dtype=torch.bfloat16, device="cuda")
        assert torch.ops.wy_lib.attention_gate_pack(x, x).shape == (5, 2048)
        acc = torch.empty(3, 8, 128, 256, device="cuda")
        m = torch.empty(3, 8, 128, device="cuda")
        pos = torch.empty(3, dtype=torch.int64, device="cuda")
        out = torch.ops.wy_lib.paged_gqa_attention_decode_combine(m, m, acc, pos)
        assert out.shape == (3, 8, 256) and out.dtype == torch.bfloat16
        xg = torch.empty(7, 1024, dtype=torch.bfloat16, device="cuda")
        wg = torch.empty(5120, 1024, dtype=torch.bfloat16, device="cuda")
        assert torch.ops.wy_lib.gemm_2d(xg, wg).shape == (7, 5120)
        qb = torch.empty(9, 8, 256, dtype=torch.bfloat16, device="cuda")
        kb = torch.empty(9, 2, 256, dtype=torch.bfloat16, device="cuda")
        cache = torch.empty(4, 2, 16, 256, dtype=torch.bfloat16, device="cuda")
        out = torch.ops.wy_lib.prefill_attention_block(
            qb, kb, kb, qb, torch.empty(1, 9, dtype=torch.int32, device="cuda"),
            torch.empty(32, device="cuda"), 64, cache, cache,
            torch.empty(1, 4, dtype=torch.int32, device="cuda"),
            torch.empty(2, dtype=torch.int32, device="cuda"), 9)
        assert out.shape == (9, 2048) and out.dtype == torch.bfloat16
        qg = torch.empty(6, 16, 128, dtype=torch.bfloat16, device="cuda")
        bg = torch.empty(6, 16, device="cuda")
        o, st = torch.ops.wy_lib.gdn_recurrent_prefill_sequential(qg, qg, qg, bg, bg)
        assert o.shape == (6, 16, 128) and st.shape == (16, 128, 128)
        o, st = torch.ops.wy_lib.gdn_recurrent_prefill_sequential(
            qg, qg, qg, bg, bg, torch.empty(3, dtype=torch.int32, device="cuda"))
        assert st.shape == (2, 16, 128, 128) and st.dtype == torch.float32
        sd = torch.empty(6, 16, 128, 128, device="cuda")
        assert torch.ops.wy_lib.gdn_recurrent_decode(qg, qg, qg, bg, bg, sd).shape == (6, 16, 128)


def test_gemm_2d_asserts_reference_preconditions(pkg):
    # the op body's assertions (gemm_2d.py:201-203) run before any launch
    body = pkg.gemm_2d._init_fn
    x = torch.zeros(2, 200, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):  # K % 128
        body(x, torch.zeros(4, 200, dtype=torch.bfloat16))
    with pytest.raises(AssertionError):  # dtype
        body(torch.zeros(2, 256), torch.zeros(4, 256))
    with pytest.raises(AssertionError):  # K mismatch
        body(torch.zeros(2, 256, dtype=torch.bfloat16), torch.zeros(4, 128, dtype=torch.bfloat16))
    with pytest.raises(Exception):  # CUDA-only op
        pkg.gemm_2d(torch.zeros(2, 256, dtype=torch.bfloat16),
                    torch.zeros(4, 256, dtype=torch.bfloat16))


def test_install_as_triton_kernels_maps_modules(pkg):
    import sys
    import types

    pkg.install_as_triton_kernels()
    for name in ("gemm_2d", "qwen_rmsnorm", "partial_rope", "attention_gate_pack",
                 "gqa_attention_decode_paged", "gqa_attention_varlen_causal"):
        mod = sys.modules[f"triton_kernels.{name}"]
        assert isinstance(mod, types.ModuleType), name
    assert hasattr(sys.modules["triton_kernels.gemm_2d"], "call_gemm_2d_triton")
    assert hasattr(sys.modules["engine.paging"], "PagePool")


# ------------------------------------------------------------------ host paging

def test_page_pool_and_sequence_pages(pkg):
    pool = pkg.PagePool(10)
    sp = pkg.SequencePages(4, batch=2, device="cpu")
    sp.reserve(17, pool, seq=0)            # 2 pages from the tail: [8, 9]
    assert sp.pages[0] == [8, 9] and sp.block_table[0, :2].tolist() == [8, 9]
    sp.reserve(20, pool, seq=0)            # still 2 pages: no-op
    assert pool.num_free == 8
    sp.reserve(48, pool, seq=1)
    assert sp.capacity(1) == 48 and pool.num_free == 5
    with pytest.raises(AssertionError):
        sp.reserve(16 * 5, pool, seq=1)    # beyond block-table capacity
    sp.release(pool)
    assert pool.num_free == 10 and int(sp.block_table.abs().sum()) == 0
    with pytest.raises(AssertionError):
        pool.alloc(11)


def test_page_pool_contract(pkg):
    """Tail-first allocation, free appends at the tail, so an alloc/free cycle
    hands back the same ids; reset restores the initial order; over-allocation
    is an AssertionError raised on the host (engine/paging.py:71-103)."""
    pool = pkg.PagePool(6)
    assert pool.alloc(0) == [] and pool.num_free == 6
    a = pool.alloc(2)
    assert a == [4, 5] and pool.num_free == 4
    b = pool.alloc(3)
    assert b == [1, 2, 3]
    pool.free(a)
    assert pool.alloc(2) == a                 # same ids after a cycle
    pool.free(b)
    pool.free([])
    assert pool.num_free == 4 and pool.alloc(1) == [3]
    with pytest.raises(AssertionError):
        pool.alloc(4)
    pool.reset()
    assert pool.num_free == 6 and pool.alloc(6) == [0, 1, 2, 3, 4, 5]


def test_sequence_pages_contract_random_walk(pkg):
    """Random reserve/release sequence against a list model of the reference's
    semantics: reserve takes only the missing pages (from the pool's tail),
    the device table row equals the held pages, release of one row returns
    its pages in row order and zeroes only that row."""
    gen = np.random.default_rng(3)
    B, max_pages = 4, 6
    pool = pkg.PagePool(20)
    sp = pkg.SequencePages(max_pages, batch=B, device="cpu")
    free_model = list(range(20))
    held_model = [[] for _ in range(B)]
    for _ in range(300):
        b = int(gen.integers(B))
        if gen.random() < 0.7:
            tokens = int(gen.integers(0, max_pages * 16 + 1))
            need = -(-tokens // 16)
            missing = need - len(held_model[b])
            if missing > len(free_model):
                with pytest.raises(AssertionError):
                    sp.reserve(tokens, pool, seq=b)
                continue
            sp.reserve(tokens, pool, seq=b)
            if missing > 0:
                held_model[b] += free_model[-missing:]
                del free_model[-missing:]
        else:
            sp.release(pool, seq=b)
            free_model += held_model[b]
            held_model[b] = []
        assert sp.pages == held_model
        assert pool.num_free == len(free_model)
        for r in range(B):
            row = sp.block_table[r].tolist()
            n = len(held_model[r])
            assert row[:n] == held_model[r] and not any(row[n:])
            assert sp.capacity(r) == 16 * n
    with pytest.raises(AssertionError):
        sp.reserve(max_pages * 16 + 1, pool, seq=0)
    sp.release(pool)
    assert pool.num_free == 20 and not sp.block_table.any()


def test_physical_rows_matches_page_layout(pkg):
    """physical_rows(bt, t, H) addresses token t, head h of a pool through
    kc.view(-1, D): checked by direct indexing kc[bt[t // 16], h, t % 16] on a
    shuffled table and against the oracle's row_index."""
    gen = torch.Generator().manual_seed(4)
    H, D, npages = 2, 8, 12
    kc = torch.randn(npages, H, 16, D, generator=gen)
    bt = torch.randperm(npages, generator=gen)[:7].to(torch.int32)
    t = torch.tensor([0, 1, 15, 16, 17, 50, 111], dtype=torch.int64)
    rows = pkg.physical_rows(bt, t, H)
    assert rows.shape == (len(t), H) and rows.dtype == torch.int64
    flat = kc.view(-1, D)
    for i, ti in enumerate(t.tolist()):
        for h in range(H):
            assert torch.equal(flat[rows[i, h]], kc[int(bt[ti // 16]), h, ti % 16])
            assert int(rows[i, h]) == orc.row_index(bt, ti, h, H)


def test_attn_caches_sizing(pkg):
    c = pkg.allocate_attn_caches(2, 100, batch=3, device="cpu")
    assert c.k_caches[0].shape == (3 * 8, 2, 16, 256)   # (ceil(100/16)+1) * 3 pages
    assert c.split_scratch[2].shape == (3, 8, 128, 256)
    c.reserve(100)
    with pytest.raises(AssertionError):
        c.reserve(101)
    c.reset()
    assert c.page_pool.num_free == 24


def test_build_packed_batch(pkg):
    pb = pkg.build_packed_batch([3, 6, 2], device="cpu")
    assert pb.cu_seqlens.tolist() == [0, 3, 9, 11]
    assert pb.position_ids.tolist() == [[0, 1, 2, 0, 1, 2, 3, 4, 5, 0, 1]]
    assert pb.slice_of(1) == slice(3, 9) and pb.max_seqlen == 6


# ------------------------------------------------------------------ fixtures

def _golden():
    return np.load(ROOT / "tests" / "golden" / "golden.npz", allow_pickle=False)


def test_golden_inputs_regenerate_bit_identically():
    g = _golden()
    d = C.decode_case()
    assert str(g["decode_inputs_sha"]) == C.digest(*d.values())
    p = C.prefill_case()
    assert str(g["prefill_inputs_sha"]) == C.digest(p["q"], p["k"], p["v"], p["cu"])
    r = C.rope_case()
    assert str(g["rope_inputs_sha"]) == C.digest(r["x"], r["pos"], r["inv_freq"])
    gg = C.gate_case()
    assert str(g["gate_inputs_sha"]) == C.digest(gg["x"], gg["gate"])
    f = C.fill_case()
    assert str(g["fill_inputs_sha"]) == C.digest(f["k"], f["v"], f["kc"], f["vc"], f["bt"], f["cu"])


def test_oracle_reproduces_golden():
    g = _golden()
    d = C.decode_case()
    kc, vc = d["kc"].clone(), d["vc"].clone()
    orc.paged_kv_append(kc, vc, d["kn"], d["vn"], d["bt"], d["pos"])
    assert str(g["decode_pool_after_sha"]) == C.digest(kc, vc)
    np.testing.assert_allclose(orc.paged_decode(d["q"], kc, vc, d["bt"], d["pos"] + 1).numpy(),
                               g["decode_out"], rtol=1e-5, atol=1e-5)
    p = C.prefill_case()
    np.testing.assert_allclose(orc.varlen_causal(p["q"], p["k"], p["v"], p["cu"]).numpy(),
                               g["prefill_out"], rtol=1e-5, atol=1e-5)
    f = C.fill_case()
    kc, vc = f["kc"].clone(), f["vc"].clone()
    orc.paged_kv_fill_varlen(kc, vc, f["k"], f["v"], f["bt"], f["cu"])
    assert str(g["fill_pool_after_sha"]) == C.digest(kc, vc)


def test_ctypes_signatures_match_header():
    """Every ctypes binding has as many arguments as its header declaration."""
    import re

    from importlib import import_module

    import __graft_entry__

    __graft_entry__.load_package()
    lib = import_module("qwen35_amd._lib")
    text = (ROOT / "include" / "wy_attn.h").read_text()
    decls = dict(re.findall(r"^(?:int|size_t|const char \*)\s*(wy_\w+)\(([^;]*)\);", text, re.M | re.S))
    for name, argtypes in lib._SIGNATURES.items():
        assert name in decls, name
        params = [p for p in decls[name].split(",") if p.strip()]
        assert len(params) == len(argtypes), (name, len(params), len(argtypes))


def test_multi_instruction_asm_outputs_are_early_clobber():
    """An inline-asm block of several instructions whose outputs are written
    asynchronously (scalar or vector memory loads) must mark every output
    early-clobber ("=&"): otherwise the compiler may give an output the
    registers of a later instruction's input, and that input is read after the
    earlier instruction's result may have landed.  (Unmarked, the decode
    step's pos / block-table pair of scalar loads got the first load's
    destination on the second load's address and faulted now and then.)"""
    import re

    for f in sorted((ROOT / "qwen3_5-triton-inference-engine_amd" / "csrc").glob("*.hip")):
        text = f.read_text()
        for m in re.finditer(r"asm\s+volatile\s*\((.*?)\);", text, re.S):
            body = m.group(1)
            parts = body.split(":")
            insts = parts[0]
            if "\\n" not in insts or len(parts) < 2:
                continue
            outs = re.findall(r'"(=[^"]*)"', parts[1])
            for o in outs:
                assert o.startswith("=&"), (f.name, body[:80], o)
