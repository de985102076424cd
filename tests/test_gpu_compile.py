"""The ops under torch.compile, as the reference runner uses them: it compiles
its forward by default (engine/runner.py:157-178), and a mutating op that
returns nothing is dropped or reordered by the compiler unless its schema
declares the mutation (triton_kernels/gqa_attention_decode_paged.py:169-173).

A function running the prefill attention (partial RoPE of q and k, varlen
causal attention, gate pack, K/V scatter) and then a decode step through the
three-op path (append, split, combine) and through the one-launch step is
compiled with fullgraph=True (no graph breaks: every op traced through its
schema and fake) and must give the eager outputs and page pools bit for bit.
A compiled function whose only effect is a void op must still write the pool.
Backend aot_eager: the graph runs the ops themselves, the check is about
tracing, functionalisation and ordering, not about generated kernels."""

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D, P = 8, 2, 256, 16
ops = torch.ops.wy_lib


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make(pkg, dev, lengths, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    bf = lambda *s: torch.randn(*s, device=dev, generator=g).to(torch.bfloat16)
    T, B = sum(lengths), len(lengths)
    max_pages = -(-(max(lengths) + 1) // P) + 1
    num_pages = B * max_pages
    bt = torch.randperm(num_pages, device=dev, generator=g).view(B, max_pages).to(torch.int32)
    packed = pkg.build_packed_batch(lengths, device=dev)
    return dict(
        q=bf(T, HQ, D), k=bf(T, HKV, D), v=bf(T, HKV, D), gate=bf(T, HQ * D),
        kc=bf(num_pages, HKV, P, D), vc=bf(num_pages, HKV, P, D), bt=bt,
        cu=packed.cu_seqlens, pos_ids=packed.position_ids, max_seqlen=packed.max_seqlen,
        qn=bf(B, HQ, D), kn=bf(B, HKV, D), vn=bf(B, HKV, D), gate_d=bf(B, HQ, D),
        pos=torch.tensor(lengths, dtype=torch.int64, device=dev),
        inv=pkg.rope_inv_freq(64, 1e7, device=dev))


def forward(q, k, v, gate, kc, vc, bt, cu, pos_ids, max_seqlen, inv, qn, kn, vn, gate_d,
            pos, m, l, acc, counters):
    T = q.shape[0]
    q4 = ops.partial_rope(q.unsqueeze(0).permute(0, 2, 1, 3), pos_ids, inv, 64)
    k4 = ops.partial_rope(k.unsqueeze(0).permute(0, 2, 1, 3), pos_ids, inv, 64)
    ctx = ops.gqa_attention_varlen_causal(q4[0].permute(1, 0, 2).contiguous(),
                                          k4[0].permute(1, 0, 2).contiguous(), v, cu,
                                          max_seqlen)
    gated = ops.attention_gate_pack(ctx.permute(1, 0, 2).unsqueeze(0),
                                    gate.view(1, T, HQ, D).permute(0, 2, 1, 3))
    ops.paged_kv_fill_varlen(kc, vc, k4[0], v.permute(1, 0, 2), bt, cu, max_seqlen)
    # decode, three-op path: append, split, combine
    ops.paged_kv_append(kc, vc, kn, vn, bt, pos)
    ops.paged_gqa_attention_decode_split(qn, kc, vc, bt, m, l, acc, pos, 0)
    dec3 = ops.paged_gqa_attention_decode_combine(m, l, acc, pos)
    # decode of the next token, one launch (append at pos + 1 included)
    pos1 = pos + 1
    dec1 = ops.paged_gqa_attention_decode_fused(qn, kn, vn, kc, vc, bt, pos1, m, l, acc,
                                                counters, gate_d)
    return gated, dec3, dec1


def test_compiled_forward_equals_eager(pkg, dev):
    lengths = [5, 130, 64, 17]
    say(f"torch.compile(aot_eager, fullgraph) prefill + decode, lengths={lengths}")
    w = make(pkg, dev, lengths, 21)
    B = len(lengths)

    def run(fn):
        kc, vc = w["kc"].clone(), w["vc"].clone()
        sc = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
        m, l, acc = sc
        outs = fn(w["q"], w["k"], w["v"], w["gate"], kc, vc, w["bt"], w["cu"],
                  w["pos_ids"], w["max_seqlen"], w["inv"], w["qn"], w["kn"], w["vn"],
                  w["gate_d"], w["pos"], m, l, acc, sc.counters)
        torch.cuda.synchronize()
        return outs, kc, vc, sc.counters

    eager, kc_e, vc_e, _ = run(forward)
    torch._dynamo.reset()
    compiled = torch.compile(forward, backend="aot_eager", fullgraph=True)
    got, kc_c, vc_c, cnt = run(compiled)
    for name, a, b in zip(("prefill gated", "decode 3-op", "decode fused"), got, eager):
        assert torch.equal(a, b), name
    assert torch.equal(kc_c, kc_e) and torch.equal(vc_c, vc_e), "pools differ from eager"
    assert not torch.equal(kc_c, w["kc"]), "the scatter/append did not run"
    assert int(cnt.abs().sum()) == 0
    # a second call reuses the compiled graph and gives the same again
    got2, kc_c2, _, _ = run(compiled)
    assert all(torch.equal(a, b) for a, b in zip(got2, eager)) and torch.equal(kc_c2, kc_e)


def test_compiled_void_ops_are_not_dropped(pkg, dev):
    """Functions whose only effect is a mutating op returning nothing."""
    say("torch.compile void ops: paged_kv_append / paged_kv_fill_varlen only")
    w = make(pkg, dev, [40, 3], 22)

    def append_only(kc, vc, kn, vn, bt, pos):
        ops.paged_kv_append(kc, vc, kn, vn, bt, pos)

    def fill_only(kc, vc, k, v, bt, cu, max_seqlen):
        ops.paged_kv_fill_varlen(kc, vc, k, v, bt, cu, max_seqlen)

    torch._dynamo.reset()
    for fn, args in ((append_only, (w["kn"], w["vn"], w["bt"], w["pos"])),
                     (fill_only, (w["k"].permute(1, 0, 2), w["v"].permute(1, 0, 2), w["bt"],
                                  w["cu"], w["max_seqlen"]))):
        kc_e, vc_e = w["kc"].clone(), w["vc"].clone()
        fn(kc_e, vc_e, *args)
        kc_c, vc_c = w["kc"].clone(), w["vc"].clone()
        torch.compile(fn, backend="aot_eager", fullgraph=True)(kc_c, vc_c, *args)
        torch.cuda.synchronize()
        assert not torch.equal(kc_e, w["kc"])
        assert torch.equal(kc_c, kc_e) and torch.equal(vc_c, vc_e), fn.__name__
