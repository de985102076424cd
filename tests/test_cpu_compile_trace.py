"""torch.compile tracing of the ops on the CPU (no kernel runs): the
reference runner compiles its forward (engine/runner.py:157-178), so every op
must trace through its schema and fake with no graph break, and each void
mutating op must survive functionalisation in program order with its mutated
caches written back (triton_kernels/gqa_attention_decode_paged.py:169-173).
The GPU test of the same function checks compiled == eager bit for bit."""

import pytest
import torch
from torch._functorch.aot_autograd import aot_module_simplified

from tests.test_gpu_compile import HQ, D, forward


class _Traced(Exception):
    pass


def _trace(fn, args):
    graphs = []

    def backend(gm, example_inputs):
        def fw(g, inputs):
            graphs.append(g)

            def run(*a):
                raise _Traced()
            return run
        return aot_module_simplified(gm, example_inputs, fw_compiler=fw)

    torch._dynamo.reset()
    with pytest.raises(_Traced):
        torch.compile(fn, backend=backend, fullgraph=True)(*args)
    assert len(graphs) == 1
    return graphs[0]


def _wy_calls(g):
    """wy_lib ops in graph order, with the names of the arguments each
    functionalised call mutates."""
    out = []
    for n in g.graph.nodes:
        if n.op != "call_function":
            continue
        t = n.target
        if "auto_functionalized" in str(t):
            op = n.args[0]
            mutated = sorted(k[1:-len("_base_index")] for k in n.kwargs if k.endswith("_base_index"))
            out.append((op._schema.name, tuple(mutated)))
        elif getattr(t, "namespace", None) == "wy_lib":
            out.append((t._schema.name, ()))
    return out


def test_forward_traces_fullgraph_with_mutations_in_order(pkg):
    lengths = [5, 130]
    g = torch.Generator().manual_seed(1)
    bf = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)
    T, B = sum(lengths), len(lengths)
    packed = pkg.build_packed_batch(lengths, device="cpu")
    bt = torch.randperm(22, generator=g).view(B, 11).to(torch.int32)
    sc = pkg.allocate_split_scratch(HQ, D, batch=B, device="cpu")
    m, l, acc = sc
    args = (bf(T, 8, 256), bf(T, 2, 256), bf(T, 2, 256), bf(T, 2048), bf(22, 2, 16, 256),
            bf(22, 2, 16, 256), bt, packed.cu_seqlens, packed.position_ids, packed.max_seqlen,
            pkg.rope_inv_freq(64, 1e7, device="cpu"), bf(B, 8, 256), bf(B, 2, 256),
            bf(B, 2, 256), bf(B, 8, 256), torch.tensor(lengths), m, l, acc, sc.counters)
    gm = _trace(forward, args)
    calls = _wy_calls(gm)
    assert calls == [
        ("wy_lib::partial_rope", ()),
        ("wy_lib::partial_rope", ()),
        ("wy_lib::gqa_attention_varlen_causal", ()),
        ("wy_lib::attention_gate_pack", ()),
        ("wy_lib::paged_kv_fill_varlen", ("k_cache", "v_cache")),
        ("wy_lib::paged_kv_append", ("k_cache", "v_cache")),
        ("wy_lib::paged_gqa_attention_decode_split", ("acc_partial", "l_partial", "m_partial")),
        ("wy_lib::paged_gqa_attention_decode_combine", ()),
        ("wy_lib::paged_gqa_attention_decode_fused",
         ("acc_partial", "counters", "k_cache", "l_partial", "m_partial", "v_cache")),
    ], calls
    # the graph returns the final value of every mutated input (k/v caches,
    # m/l/acc, counters) ahead of the three user outputs, so they are copied back
    out_node = next(n for n in gm.graph.nodes if n.op == "output")
    assert len(out_node.args[0]) == 6 + 3


def test_void_op_alone_is_kept(pkg):
    g = torch.Generator().manual_seed(2)
    bf = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)
    kc, vc = bf(8, 2, 16, 256), bf(8, 2, 16, 256)
    bt = torch.arange(8, dtype=torch.int32).view(2, 4)

    def append_only(kc, vc, kn, vn, bt, pos):
        torch.ops.wy_lib.paged_kv_append(kc, vc, kn, vn, bt, pos)

    gm = _trace(append_only, (kc, vc, bf(2, 2, 256), bf(2, 2, 256), bt, torch.tensor([3, 40])))
    assert _wy_calls(gm) == [("wy_lib::paged_kv_append", ("k_cache", "v_cache"))]
    out_node = next(n for n in gm.graph.nodes if n.op == "output")
    assert len(out_node.args[0]) == 2
